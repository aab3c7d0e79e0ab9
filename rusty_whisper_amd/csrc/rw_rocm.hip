// rw_rocm.hip -- librw_rocm.so: the C ABI of include/rw_rocm.h over the
// gfx950 kernels of rw_kernels.hpp.
//
// Host-side responsibilities (the parts of src/quant.rs that are not
// arithmetic):
//   - argument checks with the reference's failure conditions
//     (k % 32, inner-dimension mismatch, unknown dtype: src/quant.rs:757-758,
//     129) reported as status codes + per-thread error text;
//   - one-time upload + repack of a weight (QTensor::new plus the packed int8
//     cache, src/quant.rs:553-563, 589-639);
//   - regime dispatch (src/quant.rs:754-1051 picks tiers by CPU; here m
//     picks the kernel: m <= 8 -> k_gemv, else k_quantize_f16 + k_gemm);
//   - thread safety: host-pointer calls borrow a (stream, buffers) context
//     from a per-device pool, so concurrent callers never share buffers.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <stdarg.h>
#include <stdlib.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <tuple>
#include <vector>

#include "rw_attn.hpp"
#include "rw_kernels.hpp"
#include "rw_dec.hpp"
#include "rw_pool.hpp"
#include "rw_rocm.h"

using namespace rw;

// ------------------------------------------------------------- errors

static thread_local std::string g_err;

// the error text of a failure raised outside this file (rw_model.cpp)
int rw_internal_fail(int code, const char *msg) {
  g_err = msg;
  return code;
}

static int fail(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

#define HIP_TRY(expr)                                                                       \
  do {                                                                                      \
    hipError_t e_ = (expr);                                                                 \
    if (e_ != hipSuccess) return fail(RW_EHIP, "%s: %s", #expr, hipGetErrorString(e_));     \
  } while (0)

#define LAUNCH_TRY(what)                                                                    \
  do {                                                                                      \
    hipError_t e_ = hipGetLastError();                                                      \
    if (e_ != hipSuccess) return fail(RW_EHIP, "launch of %s: %s", what, hipGetErrorString(e_)); \
  } while (0)

static int bb_of(int dtype) {
  switch (dtype) {
    case RW_Q4_0: return 18;
    case RW_Q4_1: return 20;
    case RW_Q5_0: return 22;
    case RW_Q5_1: return 24;
    case RW_Q8_0: return 34;
    default: return -1;
  }
}

static size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }
static bool al16(const void *p) { return ((uintptr_t)p & 15) == 0; }
static size_t cdiv(size_t a, size_t b) { return (a + b - 1) / b; }

// ------------------------------------------------------------ devices

static std::mutex g_dev_mu;
static std::map<int, bool> g_dev_ok;  // device -> is gfx950

static int check_device(int dev) {
  std::lock_guard<std::mutex> lk(g_dev_mu);
  auto it = g_dev_ok.find(dev);
  if (it == g_dev_ok.end()) {
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, dev) != hipSuccess) return fail(RW_ENODEV, "no HIP device %d", dev);
    bool ok = strncmp(p.gcnArchName, "gfx950", 6) == 0;
    it = g_dev_ok.emplace(dev, ok).first;
    if (!ok) return fail(RW_ENODEV, "device %d is %s, this library is built for gfx950 only", dev, p.gcnArchName);
  }
  if (!it->second) return fail(RW_ENODEV, "device %d is not gfx950", dev);
  return RW_OK;
}

static int current_device(int *dev) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return fail(RW_ENODEV, "no HIP device visible");
  HIP_TRY(hipGetDevice(dev));
  return check_device(*dev);
}

// ------------------------------------------------------------ weights

struct rw_weight {
  int dtype, device;
  size_t n, k;
  int nb, nb_pad, noct, ngroups;
  void *base;
  size_t bytes;
  WeightView view;
  GemmPlanes gemm;
};

// ------------------------------------------------------ context pool

struct Ctx {
  int device;
  hipStream_t stream;
  void *buf;
  size_t cap;
};

static std::mutex g_pool_mu;
static std::vector<Ctx *> g_pool;

static int ctx_acquire(int device, Ctx **out) {
  {
    std::lock_guard<std::mutex> lk(g_pool_mu);
    for (size_t i = 0; i < g_pool.size(); ++i)
      if (g_pool[i]->device == device) {
        *out = g_pool[i];
        g_pool.erase(g_pool.begin() + i);
        return RW_OK;
      }
  }
  Ctx *c = new Ctx{device, nullptr, nullptr, 0};
  hipError_t e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete c;
    return fail(RW_EHIP, "hipStreamCreateWithFlags: %s", hipGetErrorString(e));
  }
  *out = c;
  return RW_OK;
}

static void ctx_release(Ctx *c) {
  std::lock_guard<std::mutex> lk(g_pool_mu);
  g_pool.push_back(c);
}

static int ctx_reserve(Ctx *c, size_t bytes) {
  if (c->cap >= bytes) return RW_OK;
  if (c->buf) HIP_TRY(hipFree(c->buf));
  c->buf = nullptr;
  c->cap = 0;
  size_t want = align_up(bytes < ((size_t)1 << 20) ? ((size_t)1 << 20) : bytes, (size_t)1 << 20);
  if (hipMalloc(&c->buf, want) != hipSuccess) {
    (void)hipGetLastError();
    return fail(RW_ENOMEM, "hipMalloc(%zu) for a call workspace failed", want);
  }
  c->cap = want;
  return RW_OK;
}

struct CtxGuard {
  Ctx *c = nullptr;
  ~CtxGuard() {
    if (c) ctx_release(c);
  }
};

// Per-(device, stream) workspaces for the device-pointer entries called
// without a caller workspace.  The caller holds its stream's buffer until its
// launches are queued (rw_pool.hpp): no other thread frees or grows it
// meanwhile, and launches of two threads on one stream never interleave
// over it.
using StreamKey = std::pair<int, void *>;
using WsPool = WorkspacePool<StreamKey>;
using WsHold = HoldWs<WsPool>;

static int ws_alloc(size_t bytes, void **out) {
  if (hipMalloc(out, bytes) != hipSuccess) {
    (void)hipGetLastError();
    return RW_ENOMEM;
  }
  return RW_OK;
}
static void ws_free(void *p) { (void)hipFree(p); }
static WsPool &ws_pool() {
  static WsPool *pool = new WsPool(ws_alloc, ws_free, (size_t)1 << 20);  // lives until the process ends
  return *pool;
}

static int stream_workspace(int device, void *stream, size_t bytes, WsHold &hold, void **out) {
  WsPool::Slot *slot = nullptr;
  if (ws_pool().acquire(std::make_pair(device, stream), bytes, &slot))
    return fail(RW_ENOMEM, "hipMalloc(%zu) for a stream workspace failed", bytes);
  hold.pool = &ws_pool();
  hold.slot = slot;
  *out = slot->p;
  return RW_OK;
}

// The workspace of rw_rocm_matmul_t_q_dev_noalloc: a fixed array in device
// memory that every GPU running this library holds until the process ends
// (no hipMalloc at call time).  Host code never passes `scratch` itself to a
// kernel -- its host-side name is only a handle -- but the device address
// hipGetSymbolAddress returns for the current device, taken once per device.
static __device__ __align__(256) uint8_t scratch[RW_NOALLOC_SCRATCH_BYTES];

static std::mutex g_scratch_mu;
static std::map<int, void *> g_scratch_ptr;  // device -> address of its scratch

// with `device` current
static int scratch_setup(int device, void **out) {
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  auto it = g_scratch_ptr.find(device);
  if (it == g_scratch_ptr.end()) {
    void *ptr = nullptr;
    hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      (void)hipGetLastError();
      return fail(RW_EHIP, "hipGetSymbolAddress(scratch) on device %d: %s", device, hipGetErrorString(e));
    }
    it = g_scratch_ptr.emplace(device, ptr).first;
  }
  if (out) *out = it->second;
  return RW_OK;
}

// ----------------------------------------------- activation workspace

// Products with m <= GEMV_MAX_M read the int8 layout (qa, da, pa, sa); the
// encoder GEMM reads the f16 layout (a16, rs).  The layout depends on (m, k)
// alone; the validation entries always use the int8 one.
constexpr size_t GEMV_MAX_M = 8;

struct ActLayout {
  int nb, mgroups;
  bool f16;
  size_t off_qa, off_da, off_pa, off_sa, off_a16, off_rs, off_ps, bytes;
};

static ActLayout act_layout_kind(size_t m, size_t k, bool f16) {
  ActLayout L;
  L.nb = (int)(k / QK);
  L.mgroups = (int)cdiv(m, RG);
  L.f16 = f16;
  size_t rows = (size_t)L.mgroups * RG;
  size_t nsc = rows * L.nb;
  L.off_qa = L.off_da = L.off_pa = L.off_sa = L.off_a16 = L.off_rs = L.off_ps = 0;
  if (f16) {
    L.off_a16 = 0;
    L.off_rs = align_up(rows * k * 2, 256);
    L.off_ps = align_up(L.off_rs + rows * 4, 256);
    L.bytes = align_up(L.off_ps + rows * 4, 256);
  } else {
    L.off_qa = 0;
    L.off_da = align_up(rows * k, 256);
    L.off_pa = align_up(L.off_da + nsc * 4, 256);
    L.off_sa = align_up(L.off_pa + nsc * 4, 256);
    L.bytes = align_up(L.off_sa + nsc * 4, 256);
  }
  return L;
}

static ActLayout act_layout(size_t m, size_t k) { return act_layout_kind(m, k, m > GEMV_MAX_M); }

static ActView act_view(const ActLayout &L, void *ws) {
  char *b = (char *)ws;
  ActView v{nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, L.nb, L.mgroups};
  if (L.f16) {
    v.a16 = (const uint16_t *)(b + L.off_a16);
    v.rs = (const float *)(b + L.off_rs);
    v.ps = (const float *)(b + L.off_ps);
  } else {
    v.qa = (const int8_t *)(b + L.off_qa);
    v.da = (const float *)(b + L.off_da);
    v.pa = (const float *)(b + L.off_pa);
    v.sa = (const int32_t *)(b + L.off_sa);
  }
  return v;
}

// --------------------------------------------------------- launches

static int launch_quantize(const float *a, size_t m, size_t k, const ActLayout &L, void *ws, hipStream_t s,
                           const float *lnw = nullptr, const float *lnb = nullptr) {
  char *b = (char *)ws;
  if (lnw && (!L.f16 || (L.nb + 7) / 8 > 32))
    return fail(RW_EINVAL, "layernorm + quantize takes m > %d rows of at most 8192 values", GEMV_MAX_M);
  if (L.f16) {
    if ((size_t)L.mgroups * RG * k * 2 >= ((size_t)1 << 32))
      return fail(RW_EINVAL, "activation [%zu, %zu] too large for the GEMM layout's 32-bit offsets", m, k);
    // WPR wavefronts per row, 4 / WPR rows per workgroup; NP passes of 8
    // blocks per wavefront in registers (longer rows are read twice)
    const size_t g8 = align_up((size_t)L.mgroups, 8);  // row groups, padded to whole XCD rounds
    uint16_t *a16 = (uint16_t *)(b + L.off_a16);
    float *rs = (float *)(b + L.off_rs), *ps = (float *)(b + L.off_ps);
#define RW_QF16(NP, WPR, LN)                                                                                \
  hipLaunchKernelGGL((k_quantize_f16<NP, WPR, LN>), dim3((unsigned)(g8 * RG * WPR / 4)), dim3(256), 0, s, a,     \
                     (int)m, (int)k, L.nb, a16, rs, ps, lnw, lnb)
    // The shape follows k alone, so a row's bits never depend on m.  The
    // kernel is VALU-bound (every lane of a wavefront runs a pass, live
    // blocks or not): rows of 5-6 passes (k = 1280) take 2 wavefronts of 3
    // passes (48 block slots for 40, against 64 with 4 wavefronts of 2: 4.5
    // against 4.9 us per launch at m = 1500 in a replayed graph).
    const int passes = (L.nb + 7) / 8;
    if (lnw) {
      if (passes <= 1) RW_QF16(1, 1, true);
      else if (passes <= 2) RW_QF16(1, 2, true);
      else if (passes <= 4) RW_QF16(1, 4, true);
      else if (passes <= 6) RW_QF16(3, 2, true);
      else if (passes <= 8) RW_QF16(2, 4, true);
      else if (passes <= 20) RW_QF16(5, 4, true);
      else RW_QF16(8, 4, true);
    } else {
      // rows of 5-20 passes: the same kernels' arithmetic with 4 or 8 rows
      // per wavefront, whose stores write whole runs of the plane (m = 1500:
      // 5.5 -> 5.1 us at k = 1280, 15.2 -> 13.2 us at k = 5120, cold inputs);
      // at k = 5120 two wavefronts per part, each with half of its blocks,
      // 8 per workgroup (10.28 -> 9.85 us with inputs in the MALL; 8 rows
      // per wavefront and 16 wavefronts per workgroup 10.59 us)
#define RW_QF16R(R, NP, WPR, SW)                                                                             \
  hipLaunchKernelGGL((k_quantize_f16_rows<R, NP, WPR, SW>), dim3((unsigned)(g8 * (RG / R))), dim3(64 * WPR * SW), \
                     0, s, a, (int)m, (int)k, L.nb, a16, rs, ps)
      if (passes <= 1) RW_QF16(1, 1, false);
      else if (passes <= 2) RW_QF16(1, 2, false);
      else if (passes <= 4) RW_QF16(1, 4, false);
      else if (passes <= 6) RW_QF16R(8, 3, 2, 4);
      else if (passes <= 8) RW_QF16R(4, 2, 4, 1);
      else if (passes <= 20) RW_QF16R(4, 5, 4, 2);
      else RW_QF16(8, 4, false);
#undef RW_QF16R
    }
#undef RW_QF16
    LAUNCH_TRY("k_quantize_f16");
    return RW_OK;
  }
  size_t threads = (size_t)L.mgroups * RG * L.nb * 8;
  hipLaunchKernelGGL(k_quantize, dim3((unsigned)cdiv(threads, 256)), dim3(256), 0, s, a, (int)m, (int)k, L.nb,
                     L.mgroups, (int8_t *)(b + L.off_qa), (float *)(b + L.off_da), (float *)(b + L.off_pa),
                     (int32_t *)(b + L.off_sa));
  LAUNCH_TRY("k_quantize");
  return RW_OK;
}

// The f16 activation plane (rs, ps) of rows that a GEMM_QUANT epilogue
// quantized into q ([m][k] int8) and am ([m][k / 32] block maxima):
// k_quantize_finish with the NP / WPR launch_quantize gives the same k, so
// the plane is bitwise launch_quantize's for the f32 rows.
static int launch_quantize_finish(const int8_t *q, const float *am, size_t m, size_t k, const ActLayout &L, void *ws,
                                  hipStream_t s) {
  char *b = (char *)ws;
  if (!L.f16) return fail(RW_EINVAL, "the fused quantization takes m > %d rows", GEMV_MAX_M);
  if ((size_t)L.mgroups * RG * k * 2 >= ((size_t)1 << 32))
    return fail(RW_EINVAL, "activation [%zu, %zu] too large for the GEMM layout's 32-bit offsets", m, k);
  const size_t g8 = align_up((size_t)L.mgroups, 8);
  uint16_t *a16 = (uint16_t *)(b + L.off_a16);
  float *rs = (float *)(b + L.off_rs), *ps = (float *)(b + L.off_ps);
#define RW_QFIN(NP, WPR)                                                                                   \
  hipLaunchKernelGGL((k_quantize_finish<NP, WPR>), dim3((unsigned)(g8 * RG * WPR / 4)), dim3(256), 0, s, q, am, \
                     (int)m, (int)k, L.nb, a16, rs, ps)
  const int passes = (L.nb + 7) / 8;
  if (passes <= 1) RW_QFIN(1, 1);
  else if (passes <= 2) RW_QFIN(1, 2);
  else if (passes <= 4) RW_QFIN(1, 4);
  else if (passes <= 6) RW_QFIN(3, 2);
  else if (passes <= 8) RW_QFIN(2, 4);
  else if (passes <= 20) RW_QFIN(5, 4);
  else RW_QFIN(8, 4);
#undef RW_QFIN
  LAUNCH_TRY("k_quantize_finish");
  return RW_OK;
}

// Bytes after the next product's activation layout (m rows, k = n) that the
// fused GELU + quantization keeps its int8 quants and block maxima in
static size_t fused_quant_bytes(size_t m, size_t n) {
  const size_t rows = cdiv(m, RG) * RG;
  return align_up(rows * n, 256) + align_up(rows * (n / QK) * 4, 256);
}

#define RW_DISPATCH_DT(dt, FN, ...)                  \
  switch (dt) {                                      \
    case RW_Q4_0: FN<RW_Q4_0>(__VA_ARGS__); break;   \
    case RW_Q4_1: FN<RW_Q4_1>(__VA_ARGS__); break;   \
    case RW_Q5_0: FN<RW_Q5_0>(__VA_ARGS__); break;   \
    case RW_Q5_1: FN<RW_Q5_1>(__VA_ARGS__); break;   \
    default: FN<RW_Q8_0>(__VA_ARGS__); break;        \
  }

// GEMM: a workgroup tile is 4 activation row groups x 2 weight row groups
// (128 x 64) with KW wavefronts along k.  KW is chosen from the launch's
// column tiles so that a 1500-row input (12 row tiles) gives about one
// wavefront per SIMD or more -- 1 from 48 column tiles up, 2 from 24, else 4
// -- and every wavefront keeps at least 4 blocks.  It depends on the weights
// alone, so a row's result never depends on m.
static int gemm_kw(size_t tiles, int nb) {
  int kw = tiles >= 48 ? 1 : tiles >= 24 ? 2 : 4;
  while (kw > 1 && nb < 4 * kw) kw /= 2;
  return kw;
}

// Row groups per workgroup: 4, or 2 for inputs of at most 64 rows (so a
// skinny input does not run MFMAs on repeated rows).  OFFS: some weight of
// the launch has offset rows (the epilogue's extra term and loads).
template <int DT, int KW, int TM, bool OFFS, int TN = GEMM_TN>
static void launch_gemm_tm(const GemmSet &set, size_t tiles, const ActView &av, int m, hipStream_t s) {
  dim3 grid((unsigned)tiles, (unsigned)cdiv(av.mgroups, TM));
  const GemmPlanes &g0 = set.it[0].gp;
  hipLaunchKernelGGL((k_gemm<DT, KW, TM, OFFS, TN>), grid, dim3(64 * KW), 0, s, av.a16, g0.q8, g0.dm, set.nb,
                     set.nb_pad, av.mgroups, set.it[0].ngroups, m, set.count, (int)grid.x, (int)grid.y, set, av);
}

// A skinny launch (64-row tiles that still give fewer than GEMM_TN1_BELOW
// wavefronts: the M = 40 decoder products run 60-80) takes 32-column tiles,
// twice the wavefronts.  The launch's column tiles are recounted for one
// weight row group each; the k split stays the one chosen from the weights.
#ifndef GEMM_TN1_BELOW
#define GEMM_TN1_BELOW 512
#endif
template <int DT, int KW, bool OFFS>
static bool launch_gemm_narrow(GemmSet set, size_t tiles, const ActView &av, int m, hipStream_t s) {
  if (cdiv(av.mgroups, 2) * tiles * KW >= GEMM_TN1_BELOW) return false;
  size_t t1 = 0;
  for (int i = 0; i < set.count; ++i) {
    set.it[i].tile0 = (int)t1;
    t1 += (size_t)set.it[i].ngroups;
  }
  launch_gemm_tm<DT, KW, 2, OFFS, 1>(set, t1, av, m, s);
  return true;
}

// A single-wavefront launch whose 128-row tiles leave SIMDs idle takes
// 96-row tiles when those still fit one wavefront per SIMD (q/k/v of a
// 1500-row input: 720 wavefronts of 128 rows, or 960 of 96, on 1024 SIMDs).
// A launch that 128-row tiles would give fewer than GEMM_TM2_BELOW
// wavefronts (a skinny input: a 224-row prompt's products run 120-160)
// takes 64-row tiles, twice the wavefronts (the 32 large-v3 layers'
// linears at M = 200: 2.94 -> 2.43 ms).  Tile rows change which rows share
// a workgroup, not how a row is summed.
constexpr size_t GEMM_SIMDS = 1024;
#ifndef GEMM_TM2_BELOW
#define GEMM_TM2_BELOW 512
#endif
static int gemm_rows(int kw, size_t tiles, int mgroups) {
  if (mgroups <= 2) return 2;
  if (cdiv(mgroups, 4) * tiles * kw < GEMM_TM2_BELOW) return 2;
  if (kw == 1 && cdiv(mgroups, 3) * tiles <= GEMM_SIMDS && cdiv(mgroups, 4) * tiles < cdiv(mgroups, 3) * tiles)
    return 3;
  return 4;
}

template <int DT, int KW>
static void launch_gemm_kw(const GemmSet &set, size_t tiles, const ActView &av, int m, hipStream_t s) {
  bool offs = false;
  for (int i = 0; i < set.count; ++i) offs = offs || set.it[i].gp.cm != nullptr;
  const int tm = gemm_rows(KW, tiles, av.mgroups);
  if (tm == 2 && (offs ? launch_gemm_narrow<DT, KW, true>(set, tiles, av, m, s)
                      : launch_gemm_narrow<DT, KW, false>(set, tiles, av, m, s)))
    return;
  if (offs) {
    if (tm == 2) launch_gemm_tm<DT, KW, 2, true>(set, tiles, av, m, s);
    else if (KW == 1 && tm == 3) launch_gemm_tm<DT, 1, 3, true>(set, tiles, av, m, s);
    else launch_gemm_tm<DT, KW, 4, true>(set, tiles, av, m, s);
  } else {
    if (tm == 2) launch_gemm_tm<DT, KW, 2, false>(set, tiles, av, m, s);
    else if (KW == 1 && tm == 3) launch_gemm_tm<DT, 1, 3, false>(set, tiles, av, m, s);
    else launch_gemm_tm<DT, KW, 4, false>(set, tiles, av, m, s);
  }
}

template <int DT>
static void launch_gemm_dt(const GemmSet &set, size_t tiles, const ActView &av, int m, hipStream_t s) {
  switch (gemm_kw(tiles, set.nb)) {
    case 4: launch_gemm_kw<DT, 4>(set, tiles, av, m, s); break;
    case 2: launch_gemm_kw<DT, 2>(set, tiles, av, m, s); break;
    default: launch_gemm_kw<DT, 1>(set, tiles, av, m, s); break;
  }
}

// one k_gemm launch for `count` (1 .. GEMM_MAX_SET) weights of one dtype and
// k against the quantized activation `av`.  The kernel addresses each plane
// with 32-bit byte offsets (buffer loads), so every plane stays below 4 GiB.
static int run_gemm(const rw_weight *const *w, const float *const *bias, float *const *out, size_t count,
                    const ActView &av, int m, hipStream_t s, const int *flags = nullptr, int8_t *qo = nullptr,
                    float *ao = nullptr) {
  const size_t lim = (size_t)1 << 32;
  if ((size_t)av.mgroups * (size_t)w[0]->nb * 2048 >= lim)
    return fail(RW_EINVAL, "activation [%d, %zu] too large for the GEMM's 32-bit offsets", m, w[0]->k);
  for (size_t i = 0; i < count; ++i)
    if ((size_t)w[i]->ngroups * (size_t)w[i]->nb_pad * 1024 >= lim)
      return fail(RW_EINVAL, "weight [%zu, %zu] too large for the GEMM's 32-bit offsets", w[i]->n, w[i]->k);
  GemmSet set{};
  set.count = (int)count;
  set.nb = w[0]->nb;
  set.nb_pad = w[0]->nb_pad;
  size_t tiles = 0;
  for (size_t i = 0; i < count; ++i) {
    GemmItem &it = set.it[i];
    it.gp = w[i]->gemm;
    it.bias = bias ? bias[i] : nullptr;
    it.out = out[i];
    it.n = (int)w[i]->n;
    it.ngroups = w[i]->ngroups;
    it.flags = flags ? flags[i] : 0;
    it.qo = qo;
    it.ao = ao;
    it.tile0 = (int)tiles;
    tiles += cdiv(w[i]->ngroups, GEMM_TN);
  }
  RW_DISPATCH_DT(w[0]->dtype, launch_gemm_dt, set, tiles, av, m, s);
  LAUNCH_TRY("k_gemm");
  return RW_OK;
}

// ------------------------------------------------------ decode GEMV

// The split of a row's octets over wavefronts depends on the weight and the
// launch form only.  Grouped launches have workgroups to spare and split
// while every wavefront keeps at least 6 octets: each workgroup copies its
// items' records for the whole k into LDS, so k = 5120 in two parts of 10
// octets instead of four of 5 halves those copies (large-v3 decoder set,
// M = 5: 5.02-5.08 -> 5.17-5.28 TB/s on one box); a single linear's launch
// is short of workgroups at decode sizes and splits while every wavefront
// keeps 2, which halves its latency.  The two forms then differ only by the
// f32 reassociation of the parts' sums.  Single and set launches also give
// each wavefront one row group instead of two (gemv_ng): a 1280-row weight
// at k = 1280 runs on 20 workgroups instead of 10 (decoder step 3.61 ->
// 2.96 ms per token).
#ifndef GEMV_SINGLE_KEEP
#define GEMV_SINGLE_KEEP 2
#endif
static int gemv_ks(const rw_weight *w, bool single = false) {
  const int keep = single ? GEMV_SINGLE_KEEP : 6;
  int ks = 1;
  while (ks < 4 && w->noct / (2 * ks) >= keep) ks *= 2;
  return ks;
}
static int gemv_wgs(const rw_weight *w, int ks, bool grouped) {
  return (int)cdiv(w->ngroups, gemv_ng(grouped) * (4 / ks));
}

// LDS per workgroup is held to GEMV_LDS_CAP bytes: activation records go
// through LDS in chunks (the arithmetic does not depend on them).  A weight
// split over ks wavefront sets needs ks * ceil(noct / ks) octet slots to hold
// its whole k at once; a launch gets the most any of its weights needs, up
// to the cap.
#ifndef GEMV_LDS_CAP
#define GEMV_LDS_CAP 32768
#endif
static int gemv_need(const rw_weight *w, bool single = false) {
  const int ks = gemv_ks(w, single);
  return ks * (int)cdiv(w->noct, ks);
}
// A single or set launch of at most GEMV_LAT_WGS workgroups (the latency
// form's candidates, one workgroup per CU) may hold twice that, so that the
// records of 5 rows over a 4-way split k = 5120 (20 octets) fit at once and
// the launch takes the latency form.
#ifndef GEMV_LDS_CAP_LAT
#define GEMV_LDS_CAP_LAT 65536
#endif
constexpr int GEMV_LAT_WGS = 256;  // 4 wavefronts each: one per SIMD of 256 CUs
static int gemv_cap(int m, int need, int wgs = 1 << 30) {
  const size_t bytes = wgs <= GEMV_LAT_WGS ? GEMV_LDS_CAP_LAT : GEMV_LDS_CAP;
  int cap = (int)(bytes / ((size_t)OCT * gemv_rec_bytes(m)));
  if (cap < 4) cap = 4;
  return need < cap ? need : cap;
}

static GemvItem gemv_item(const rw_weight *w, const float *a, const float *bias, float *out, bool single = false) {
  GemvItem it{};
  it.w = w->view;
  it.a = a;
  it.bias = bias;
  it.out = out;
  it.n = (int)w->n;
  const int ks = gemv_ks(w, single);
  it.lks = ks == 4 ? 2 : ks == 2 ? 1 : 0;
  return it;
}

// A single or set launch of at most one wavefront per SIMD whose records fit
// LDS at once takes k_gemv's latency form: every wavefront keeps up to
// GEMV_PD weight octets in flight (it has the registers of a whole SIMD).
// With one row group per wavefront three octets fit without spilling and
// cover a 1280-wide row's larger part (2 + 3 octets) in one round trip; a
// fourth measured no better.
#ifndef GEMV_PD_LAT
#define GEMV_PD_LAT 3
#endif
constexpr int GEMV_PD = GEMV_PD_LAT;
static bool gemv_latency_form(const GemvSet &one, int wgs, int cap_oct) {
  if (wgs > GEMV_LAT_WGS) return false;
  for (int i = 0; i < one.count; ++i) {
    const int lks = one.it[i].lks, span = (one.it[i].w.noct + (1 << lks) - 1) >> lks;
    if ((cap_oct >> lks) < span) return false;  // the records would come in chunks
  }
  return true;
}

template <int DT, int MR>
static void launch_gemv_mr(const GemvItem *items, const int2 *wg_item, const GemvSet &one, int wgs, int cap_oct,
                           hipStream_t s) {
  const size_t lds = gemv_lds_bytes(MR, cap_oct);
  // k_gemv's leading scalars: the first item's rows, planes and geometry
  // (zeros for a grouped launch, whose items are in the device table)
  const GemvItem &f = one.it[0];
  static_assert(GEMV_LDS_CAP_LAT / (OCT * gemv_rec_bytes(1)) < 256 && GEMV_LDS_CAP / (OCT * gemv_rec_bytes(1)) < 256,
                "k_gemv's header holds cap_oct in 8 bits");
  const int hdr = items ? 0 : one.count | f.lks << 4 | (f.lnw ? 1 : 0) << 6 | cap_oct << 8;
#define RW_GEMV_HEAD                                                                                             \
  f.a, (const uint8_t *)f.w.qs, (const uint16_t *)f.w.d, (const uint32_t *)f.w.qh, (const uint16_t *)f.w.m, f.w.nb, \
      f.w.noct, f.w.ngroups, hdr
  if (items)
    hipLaunchKernelGGL((k_gemv<DT, MR, true>), dim3((unsigned)wgs), dim3(256), lds, s, nullptr, nullptr, nullptr,
                       nullptr, nullptr, 0, 0, 0, 0, items, wg_item, one, cap_oct);
  else if (gemv_latency_form(one, wgs, cap_oct))
    hipLaunchKernelGGL((k_gemv<DT, MR, false, GEMV_PD>), dim3((unsigned)wgs), dim3(256), lds, s, RW_GEMV_HEAD,
                       items, wg_item, one, cap_oct);
  else
    hipLaunchKernelGGL((k_gemv<DT, MR, false>), dim3((unsigned)wgs), dim3(256), lds, s, RW_GEMV_HEAD, items,
                       wg_item, one, cap_oct);
#undef RW_GEMV_HEAD
}

// one k_gemv launch: `items` (device) + `wg_item` (device) for a group, or
// items == NULL and the set `one` (kernel arguments)
template <int DT>
static void launch_gemv_dt(int m, const GemvItem *items, const int2 *wg_item, const GemvSet &one, int wgs,
                           int cap_oct, hipStream_t s) {
  switch (m) {
    case 1: launch_gemv_mr<DT, 1>(items, wg_item, one, wgs, cap_oct, s); break;
    case 2: launch_gemv_mr<DT, 2>(items, wg_item, one, wgs, cap_oct, s); break;
    case 3: launch_gemv_mr<DT, 3>(items, wg_item, one, wgs, cap_oct, s); break;
    case 4: launch_gemv_mr<DT, 4>(items, wg_item, one, wgs, cap_oct, s); break;
    case 5: launch_gemv_mr<DT, 5>(items, wg_item, one, wgs, cap_oct, s); break;
    case 6: launch_gemv_mr<DT, 6>(items, wg_item, one, wgs, cap_oct, s); break;
    case 7: launch_gemv_mr<DT, 7>(items, wg_item, one, wgs, cap_oct, s); break;
    default: launch_gemv_mr<DT, 8>(items, wg_item, one, wgs, cap_oct, s); break;
  }
}

#define RW_DISPATCH_GEMV(w, m, ...)                                              \
  switch ((w)->dtype) {                                                          \
    case RW_Q4_0: launch_gemv_dt<RW_Q4_0>((int)(m), __VA_ARGS__); break;         \
    case RW_Q4_1: launch_gemv_dt<RW_Q4_1>((int)(m), __VA_ARGS__); break;         \
    case RW_Q5_0: launch_gemv_dt<RW_Q5_0>((int)(m), __VA_ARGS__); break;         \
    case RW_Q5_1: launch_gemv_dt<RW_Q5_1>((int)(m), __VA_ARGS__); break;         \
    default: launch_gemv_dt<RW_Q8_0>((int)(m), __VA_ARGS__); break;              \
  }

// the product from an already quantized workspace, on `s`
static int run_product(const rw_weight *w, size_t m, const float *bias, float *out, const void *ws,
                       hipStream_t s) {
  ActLayout L = act_layout(m, w->k);
  ActView av = act_view(L, (void *)ws);
  if (m <= GEMV_MAX_M) {
    GemvSet one{};
    one.it[0] = gemv_item(w, nullptr, bias, out, true);
    one.it[0].qa = av.qa;
    one.it[0].qda = av.da;
    one.it[0].qpa = av.pa;
    one.it[0].qsa = av.sa;
    one.count = 1;
    one.end[0] = gemv_wgs(w, gemv_ks(w, true), false);
    RW_DISPATCH_GEMV(w, m, nullptr, nullptr, one, one.end[0], gemv_cap((int)m, gemv_need(w, true), one.end[0]), s);
    LAUNCH_TRY("k_gemv");
  } else {
    return run_gemm(&w, &bias, &out, 1, av, (int)m, s);
  }
  return RW_OK;
}

// quantize + product on `s`, all pointers on the device; the decode shape
// quantizes inside its one launch and does not touch `ws`
static int run_matmul(const rw_weight *w, const float *a, size_t m, const float *bias, float *out, void *ws,
                      hipStream_t s) {
  if (m == 0) return RW_OK;
  if (m <= GEMV_MAX_M) {
    GemvSet one{};
    one.it[0] = gemv_item(w, a, bias, out, true);
    one.count = 1;
    one.end[0] = gemv_wgs(w, gemv_ks(w, true), false);
    RW_DISPATCH_GEMV(w, m, nullptr, nullptr, one, one.end[0], gemv_cap((int)m, gemv_need(w, true), one.end[0]), s);
    LAUNCH_TRY("k_gemv");
    return RW_OK;
  }
  ActLayout L = act_layout(m, w->k);
  int rc = launch_quantize(a, m, w->k, L, ws, s);
  if (rc) return rc;
  return run_product(w, m, bias, out, ws, s);
}

#define RW_TRY(expr)       \
  do {                     \
    int rc_ = (expr);      \
    if (rc_) return rc_;   \
  } while (0)

static int launch_layernorm(float *x, size_t rows, size_t n, const float *w, const float *b, float *y,
                            hipStream_t s, const float *r);

// several linears of one dtype and k on one activation a: one GEMV launch
// (kernel-argument set) at m <= 8, else one quantization and one GEMM launch.
// With lnw the rows of a are layernormed (lnw, lnb) before they are
// quantized, inside that launch; `flags` (GEMM_GELU, GEMM_ACC) go to every
// linear's epilogue.  `tmp` ([m, k] f32, or NULL) takes the layernormed rows
// where the GEMM's quantizer cannot fold the layernorm (k > 8192).
// rec_out / rec_in (decode sizes, one linear): the product also writes its
// outputs' activation records (GEMV_REC_OUT), or reads its rows as records
// another product wrote instead of quantizing `a`.
static int run_matmul_set(const rw_weight *const *w, size_t count, const float *a, size_t m,
                          const float *const *bias, float *const *out, void *ws, hipStream_t s,
                          const float *lnw = nullptr, const float *lnb = nullptr, int flags = 0,
                          float *tmp = nullptr, uint8_t *rec_out = nullptr, uint8_t *rec_in = nullptr) {
  if (m == 0) return RW_OK;
  if (count < 1 || count > (size_t)GEMV_SET) return fail(RW_EINVAL, "a set holds 1 to %d linears", GEMV_SET);
  if ((rec_out || rec_in) && (count != 1 || m < 2 || m > GEMV_MAX_M))
    return fail(RW_EINVAL, "activation records pass between single linears of 2 to %d rows", GEMV_MAX_M);
  if (m <= GEMV_MAX_M) {
    GemvSet set{};
    int wgs = 0, need = 0;
    for (size_t i = 0; i < count; ++i) {
      set.it[i] = gemv_item(w[i], a, bias ? bias[i] : nullptr, out[i], true);
      set.it[i].lnw = lnw;
      set.it[i].lnb = lnb;
      set.it[i].flags = flags;
      if (rec_out) {
        set.it[i].rec = rec_out;
        set.it[i].flags |= GEMV_REC_OUT;
      }
      if (rec_in) {
        set.it[i].a = nullptr;
        set.it[i].rec = rec_in;
      }
      wgs += gemv_wgs(w[i], gemv_ks(w[i], true), false);
      set.end[i] = wgs;
      need = std::max(need, gemv_need(w[i], true));
    }
    set.count = (int)count;
    RW_DISPATCH_GEMV(w[0], m, nullptr, nullptr, set, wgs, gemv_cap((int)m, need, wgs), s);
    LAUNCH_TRY("k_gemv");
    return RW_OK;
  }
  const size_t k = w[0]->k;
  ActLayout L = act_layout(m, k);
  if (lnw && (L.nb + 7) / 8 > 32) {  // layernorm in its own launch
    if (!tmp) return fail(RW_EINVAL, "layernorm + product over k = %zu needs a row buffer", k);
    RW_TRY(launch_layernorm(const_cast<float *>(a), m, k, lnw, lnb, tmp, s, nullptr));
    a = tmp;
    lnw = lnb = nullptr;
  }
  RW_TRY(launch_quantize(a, m, k, L, ws, s, lnw, lnb));
  const int fl[GEMV_SET] = {flags, flags, flags, flags};
  return run_gemm(w, bias, out, count, act_view(L, ws), (int)m, s, flags ? fl : nullptr);
}

// one linear (count 1) with the options of run_matmul_set
static int run_linear(const rw_weight *w, const float *a, size_t m, const float *bias, float *out, void *ws,
                      hipStream_t s, const float *lnw, const float *lnb, int flags, float *tmp,
                      uint8_t *rec_out = nullptr, uint8_t *rec_in = nullptr) {
  return run_matmul_set(&w, 1, a, m, &bias, &out, ws, s, lnw, lnb, flags, tmp, rec_out, rec_in);
}

// ------------------------------------------------- grouped decode GEMV

// A grouped call becomes, per distinct (dtype, m), one k_gemv_records launch
// (each linear's activation quantized once, into records) and one k_gemv
// launch.  The device buffer holds the item table, the workgroup -> item maps
// of both launches (these go to the device in one copy) and the records.
struct GroupLaunch {
  int dt, m, wgs, cap_oct, wg_first, qwgs, qwg_first;
};

struct GroupPlan {
  std::vector<size_t> order;    // non-empty items, in launch order
  std::vector<size_t> rec_off;  // per ordered item, from rec_base
  std::vector<GroupLaunch> launches;
  std::vector<size_t> first;    // per launch: its first ordered item
  std::vector<int2> map, qmap;  // slot -> (ordered item, tile / part), all launches
  size_t map_off = 0, qmap_off = 0;
  size_t bytes = 0;     // item table + maps (copied from the host)
  size_t rec_base = 0;  // records start
  size_t total = 0;     // bytes of device memory the group needs
};

// Workgroup slots of a grouped launch.  XCDs take workgroups round-robin
// (slot 8 p + x runs on XCD x), and each XCD's L2 serves its workgroups.
// An item's tiles go in runs of up to GEMV_RUN consecutive slots of one XCD,
// so a run reads the item's activation records through one L2; each run goes
// to the XCD with the fewest slots so far.  The records kernel's parts of an
// item all run on the XCD of the item's first run, so that run finds the
// records in its L2 (2 us less for the large-v3 decoder set at M = 5 than
// with the parts placed on their own; every run of an item on one XCD was
// 15% slower; runs of 16 rather than 8 or 4: 5.27-5.33 against 5.23-5.26
// and 5.08-5.12 TB/s at M = 5, one box; 32 no better).  Unused slots map to
// item -1.
#ifndef GEMV_RUN_SLOTS
#define GEMV_RUN_SLOTS 16
#endif
constexpr int GEMV_RUN = GEMV_RUN_SLOTS;


// Returns the XCD of the item's first run.  With `xcd` >= 0 every run goes
// to that XCD instead (the records kernel's parts of an item are written
// through the L2 of the XCD whose GEMV run reads them first).
static int place_runs(int item, int n, int *pos, std::vector<int2> &slots, int xcd = -1) {
  int first = -1;
  for (int t0 = 0; t0 < n; t0 += GEMV_RUN) {
    int x = 0;
    for (int c = 1; c < 8; ++c)
      if (pos[c] < pos[x]) x = c;
    if (xcd >= 0) x = xcd;
    if (first < 0) first = x;
    const int cnt = std::min(GEMV_RUN, n - t0);
    for (int q = 0; q < cnt; ++q) {
      const size_t slot = (size_t)8 * (pos[x] + q) + x;
      if (slots.size() <= slot) slots.resize(slot + 1, make_int2(-1, 0));
      slots[slot] = make_int2(item, t0 + q);
    }
    pos[x] += cnt;
  }
  return first;
}

static GroupPlan group_plan(const rw_linear *items, size_t count) {
  GroupPlan P;
  auto key = [&](size_t i) {
    const rw_weight *w = items[i].w;
    return std::make_tuple(w->dtype, (int)items[i].m);
  };
  for (size_t i = 0; i < count; ++i)
    if (items[i].w && items[i].m > 0 && items[i].m <= GEMV_MAX_M) P.order.push_back(i);
  std::stable_sort(P.order.begin(), P.order.end(), [&](size_t x, size_t y) { return key(x) < key(y); });
  const size_t no = P.order.size();
  P.rec_off.assign(no, 0);
  size_t rec = 0;
  for (size_t j0 = 0; j0 < no;) {
    size_t j1 = j0 + 1;
    while (j1 < no && key(P.order[j1]) == key(P.order[j0])) ++j1;
    GroupLaunch L{items[P.order[j0]].w->dtype, (int)items[P.order[j0]].m, 0, 0, (int)P.map.size(), 0,
                  (int)P.qmap.size()};
    std::vector<int2> slots, qslots;
    int pos[8] = {}, qpos[8] = {};
    // Workgroups start in slot order as earlier ones end.  Those of k-split
    // items (two or four wavefront sets along k, which meet at the end) run
    // the longest, so their slots come first and the workgroups that start
    // last, once the resident slots have turned over, are shorter ones.
    std::vector<size_t> place(j1 - j0);
    for (size_t j = j0; j < j1; ++j) place[j - j0] = j;
    std::stable_sort(place.begin(), place.end(),
                     [&](size_t x, size_t y) { return gemv_ks(items[P.order[x]].w) > gemv_ks(items[P.order[y]].w); });
    for (const size_t j : place) {
      const rw_weight *w = items[P.order[j]].w;
      const int m = (int)items[P.order[j]].m;
      const int x0 = place_runs((int)j, gemv_wgs(w, gemv_ks(w), true), pos, slots);
      place_runs((int)j, (int)cdiv((size_t)m * w->noct * OCT, 32), qpos, qslots, x0);
      P.rec_off[j] = rec;
      rec += align_up((size_t)w->noct * OCT * gemv_rec_bytes(m), 256);
      L.cap_oct = std::max(L.cap_oct, gemv_need(w));
    }
    L.wgs = (int)align_up(slots.size(), 8);
    L.qwgs = (int)align_up(qslots.size(), 8);
    slots.resize(L.wgs, make_int2(-1, 0));
    qslots.resize(L.qwgs, make_int2(-1, 0));
    P.map.insert(P.map.end(), slots.begin(), slots.end());
    P.qmap.insert(P.qmap.end(), qslots.begin(), qslots.end());
    L.cap_oct = gemv_cap(L.m, L.cap_oct);
    P.launches.push_back(L);
    P.first.push_back(j0);
    j0 = j1;
  }
  P.map_off = align_up(no * sizeof(GemvItem), 256);
  P.qmap_off = P.map_off + P.map.size() * sizeof(int2);
  P.bytes = no == 0 ? 0 : align_up(P.qmap_off + P.qmap.size() * sizeof(int2), 256);
  P.rec_base = P.bytes;
  P.total = no == 0 ? 0 : P.rec_base + rec;
  return P;
}

// a prepared group: its tables stay on the device, a run only launches
struct rw_group {
  int device;
  std::vector<GroupLaunch> launches;
  void *table;
  size_t map_off, qmap_off, bytes;
};

// pinned staging for launch tables, one per (device, stream); `ev` marks the
// end of the last copy out of it
struct Stage {
  void *host = nullptr;
  size_t cap = 0;
  hipEvent_t ev = nullptr;
  bool pending = false;
};
static std::mutex g_stage_mu;
static std::map<std::pair<int, void *>, Stage> g_stage;

static int check_matmul_args(const rw_weight *w, const void *a, size_t m, size_t k, const void *out);

static int check_group_items(const rw_linear *items, size_t count) {
  for (size_t i = 0; i < count; ++i) {
    const rw_linear &it = items[i];
    int rc = check_matmul_args(it.w, it.a, it.m, it.w ? it.w->k : 0, it.out);
    if (rc) return fail(rc, "item %zu: %s", i, g_err.c_str());
    if (it.m > GEMV_MAX_M) return fail(RW_EINVAL, "item %zu: m = %zu > %zu", i, it.m, GEMV_MAX_M);
    if (it.w->device != items[0].w->device) return fail(RW_EINVAL, "item %zu is on another device", i);
  }
  return RW_OK;
}

// item table, then the two workgroup -> item maps, as the plan lays them out;
// `dev` is the device address the tables will have (the records follow them)
static void fill_tables(const GroupPlan &P, const rw_linear *items, void *host, void *dev) {
  GemvItem *tab = (GemvItem *)host;
  for (size_t j = 0; j < P.order.size(); ++j) {
    const rw_linear &it = items[P.order[j]];
    tab[j] = gemv_item(it.w, it.a, it.bias, it.out);
    tab[j].rec = (uint8_t *)dev + P.rec_base + P.rec_off[j];
  }
  memcpy((char *)host + P.map_off, P.map.data(), P.map.size() * sizeof(int2));
  memcpy((char *)host + P.qmap_off, P.qmap.data(), P.qmap.size() * sizeof(int2));
}

template <int DT>
static void launch_records_dt(int m, const GemvItem *items, const int2 *qmap, int qwgs, hipStream_t s) {
#define RW_REC(MR)                                                                                          \
  hipLaunchKernelGGL((k_gemv_records<DT, MR>), dim3((unsigned)qwgs), dim3(256), 0, s, items, qmap)
  switch (m) {
    case 1: RW_REC(1); break;
    case 2: RW_REC(2); break;
    case 3: RW_REC(3); break;
    case 4: RW_REC(4); break;
    case 5: RW_REC(5); break;
    case 6: RW_REC(6); break;
    case 7: RW_REC(7); break;
    default: RW_REC(8); break;
  }
#undef RW_REC
}

static int launch_group(const std::vector<GroupLaunch> &launches, const void *table, size_t map_off,
                        size_t qmap_off, hipStream_t s) {
  const GemvItem *dtab = (const GemvItem *)table;
  const int2 *dmap = (const int2 *)((const char *)table + map_off);
  const int2 *qmap = (const int2 *)((const char *)table + qmap_off);
  const GemvSet none{};
  for (const GroupLaunch &L : launches) {
    switch (L.dt) {
      case RW_Q4_0: launch_records_dt<RW_Q4_0>(L.m, dtab, qmap + L.qwg_first, L.qwgs, s); break;
      case RW_Q4_1: launch_records_dt<RW_Q4_1>(L.m, dtab, qmap + L.qwg_first, L.qwgs, s); break;
      case RW_Q5_0: launch_records_dt<RW_Q5_0>(L.m, dtab, qmap + L.qwg_first, L.qwgs, s); break;
      case RW_Q5_1: launch_records_dt<RW_Q5_1>(L.m, dtab, qmap + L.qwg_first, L.qwgs, s); break;
      default: launch_records_dt<RW_Q8_0>(L.m, dtab, qmap + L.qwg_first, L.qwgs, s); break;
    }
    LAUNCH_TRY("k_gemv_records (grouped)");
    switch (L.dt) {
      case RW_Q4_0: launch_gemv_dt<RW_Q4_0>(L.m, dtab, dmap + L.wg_first, none, L.wgs, L.cap_oct, s); break;
      case RW_Q4_1: launch_gemv_dt<RW_Q4_1>(L.m, dtab, dmap + L.wg_first, none, L.wgs, L.cap_oct, s); break;
      case RW_Q5_0: launch_gemv_dt<RW_Q5_0>(L.m, dtab, dmap + L.wg_first, none, L.wgs, L.cap_oct, s); break;
      case RW_Q5_1: launch_gemv_dt<RW_Q5_1>(L.m, dtab, dmap + L.wg_first, none, L.wgs, L.cap_oct, s); break;
      default: launch_gemv_dt<RW_Q8_0>(L.m, dtab, dmap + L.wg_first, none, L.wgs, L.cap_oct, s); break;
    }
    LAUNCH_TRY("k_gemv (grouped)");
  }
  return RW_OK;
}

static int check_matmul_args(const rw_weight *w, const void *a, size_t m, size_t k, const void *out) {
  if (!w) return fail(RW_EINVAL, "weight is NULL");
  if (k != w->k) return fail(RW_EINVAL, "matmul_t_q inner dims: %zu vs %zu", k, w->k);
  if (m > 0 && (!a || !out)) return fail(RW_EINVAL, "activation or output pointer is NULL");
  if (m > (size_t)INT32_MAX / 2) return fail(RW_EINVAL, "m = %zu is too large", m);
  return RW_OK;
}

// --------------------------------------------------------------- ABI

// ------------------------------------------------------ attention

// Workspace of one attention call: the f16 pairs of q, k and v^T.
struct AttnLayout {
  int n_head, tq_pad, tkv_pad, nsplit;
  size_t off_qh, off_ql, off_kh, off_kl, off_vh, off_vl, off_part, bytes;
};

// few (query block, head) workgroups -- a decoding step: split the kv
// blocks over up to ATT_MAX_SPLIT workgroups each (down to one 32-row block
// per run: each run is then one short chain of loads; the decoder step's
// cross-attention, 47 blocks per head, runs 26 splits instead of 11: 2% per
// token, 3% at 440 cached rows), merged by k_attn_combine
#ifndef ATT_SPLIT_MINBLK
#define ATT_SPLIT_MINBLK 1
#endif
static int attn_nsplit(size_t groups, size_t nblk) {
  if (groups < 256 && nblk >= 8)
    return (int)std::min<size_t>(ATT_MAX_SPLIT, std::min<size_t>(nblk / ATT_SPLIT_MINBLK, cdiv(512, groups)));
  return 1;
}

// kv_planes = false: the call reads K/V planes split beforehand (the
// decoder's cross-attention), so the layout holds q's planes and the split
// runs' partial results only
static AttnLayout attn_layout(size_t t_q, size_t t_kv, size_t n_state, bool kv_planes = true) {
  AttnLayout L{};
  L.n_head = (int)(n_state / ATT_DH);
  L.tq_pad = (int)align_up(t_q, ATT_QB);
  L.tkv_pad = (int)align_up(t_kv, ATT_KVB);
  const size_t qb = (size_t)L.n_head * L.tq_pad * ATT_DH * 2;
  const size_t kb = kv_planes ? (size_t)L.n_head * L.tkv_pad * ATT_DH * 2 : 0;
  L.off_qh = 0;
  L.off_ql = align_up(L.off_qh + qb, 256);
  L.off_kh = align_up(L.off_ql + qb, 256);
  L.off_kl = align_up(L.off_kh + kb, 256);
  L.off_vh = align_up(L.off_kl + kb, 256);
  L.off_vl = align_up(L.off_vh + kb, 256);
  L.nsplit = attn_nsplit((size_t)(L.tq_pad / ATT_QB) * L.n_head, cdiv(t_kv, ATT_KVB));
  L.off_part = align_up(L.off_vl + kb, 256);
  const size_t part = L.nsplit > 1 ? (size_t)L.nsplit * L.n_head * L.tq_pad * (ATT_DH + 2) * 4 : 0;
  L.bytes = align_up(L.off_part + part, 256);
  return L;
}

// The reference's conditions (src/encoder.rs:48-58, 109-119) plus this
// kernel's: 64-value heads, 16-byte aligned rows.
static int check_attn_args(const float *q, size_t ldq, const float *k, size_t ldk, const float *v, size_t ldv,
                           size_t t_q, size_t t_kv, size_t n_state, int n_head, int causal, const float *out,
                           size_t ldo) {
  if (n_head <= 0 || n_state == 0 || n_state % (size_t)n_head)
    return fail(RW_EINVAL, "n_state %zu is not a positive multiple of n_head %d", n_state, n_head);
  if (n_state / (size_t)n_head != ATT_DH)
    return fail(RW_EINVAL, "head size %zu unsupported (the kernel takes %d)", n_state / (size_t)n_head, ATT_DH);
  if (causal && t_q > t_kv) return fail(RW_EINVAL, "causal attention needs t_q <= t_kv (%zu > %zu)", t_q, t_kv);
  if (t_q > (1u << 24) || t_kv > (1u << 24)) return fail(RW_EINVAL, "sequence too long");
  // k_attn packs its grid's y extent (heads, times 8 beams at most) above 8 bits of one int
  if (n_head >= (1 << 19)) return fail(RW_EINVAL, "n_head %d too large", n_head);
  if (t_q == 0) return RW_OK;
  if (!q || !out || (t_kv && (!k || !v))) return fail(RW_EINVAL, "q, k, v or out is NULL");
  if (ldq < n_state || ldk < n_state || ldv < n_state || ldo < n_state)
    return fail(RW_EINVAL, "a row stride is smaller than n_state");
  if (ldq % 4 || ldk % 4 || ldv % 4 || ldo % 4 || ((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)out) % 16)
    return fail(RW_EINVAL, "q, k, v and out rows must be 16-byte aligned");
  return RW_OK;
}

// rec (2-8 query rows): where the kv is split, the merge also writes the
// output rows' activation records for the next product (offset term
// rec_off), and *rec_done says whether it did.
static int run_attention(const float *q, size_t ldq, const float *k, size_t ldk, const float *v, size_t ldv,
                         size_t t_q, size_t t_kv, int n_head, int causal, float *out, size_t ldo, const AttnLayout &L,
                         void *ws, hipStream_t s, const AttnPlanes *kv_split = nullptr, uint8_t *rec = nullptr,
                         int rec_off = 0, bool *rec_done = nullptr) {
  if (rec_done) *rec_done = false;
  char *b = (char *)ws;
  uint16_t *qh = (uint16_t *)(b + L.off_qh), *ql = (uint16_t *)(b + L.off_ql);
  uint16_t *kh = (uint16_t *)(b + L.off_kh), *kl = (uint16_t *)(b + L.off_kl);
  uint16_t *vh = (uint16_t *)(b + L.off_vh), *vl = (uint16_t *)(b + L.off_vl);
  if (t_kv == 0) {  // no keys: every output row is the empty sum
    const size_t nz = t_q * (size_t)n_head * ATT_DH;
    hipLaunchKernelGGL(k_attn_zero, dim3((unsigned)cdiv(nz, 256)), dim3(256), 0, s, out, (int)ldo, (int)t_q,
                       n_head * ATT_DH);
    LAUNCH_TRY("k_attn_zero");
    return RW_OK;
  }
  // k_attn splits q (f32, scaled by 1/8) as it loads it; K and v^T are split
  // here, or were split before (kv_split: the decoder's cross-attention)
  // planes padded to this call's t_kv (the layout may be sized for a longer
  // one, e.g. a decoder's n_ctx)
  AttnPlanes P{qh, ql, kh, kl, vh, vl, L.tq_pad, (int)std::min<size_t>(align_up(t_kv, ATT_KVB), L.tkv_pad)};
  if (kv_split) {
    P.kh = kv_split->kh, P.kl = kv_split->kl, P.vh = kv_split->vh, P.vl = kv_split->vl;
    P.tkv_pad = kv_split->tkv_pad;
  }
  // one query block against k and v rows (a decoding step's self-attention):
  // k_attn splits q, K and V as it loads them
  const bool rows = !kv_split && L.tq_pad == ATT_QB;
  if (!kv_split && !rows) {  // k and v only: k_attn splits q as it loads it
    const size_t nk = (size_t)n_head * P.tkv_pad * 8;
    const int wk = (int)cdiv(nk, 256);
    const int wv = n_head * (int)cdiv(P.tkv_pad, ATT_VT_KV);  // v^T: one workgroup per (head, 64 positions)
    hipLaunchKernelGGL(k_attn_split, dim3((unsigned)(wk + wv)), dim3(256), 0, s, q, (int)ldq, (int)t_q, k,
                       (int)ldk, v, (int)ldv, (int)t_kv, P, n_head, 0, wk);
    LAUNCH_TRY("k_attn_split");
  }
  // this call's split (the layout's is for its longest kv; the rule grows
  // with the kv length, so this one fits the layout's part buffer)
  const int nsplit = std::min(L.nsplit, attn_nsplit((size_t)(L.tq_pad / ATT_QB) * n_head, cdiv(t_kv, ATT_KVB)));
  float *part = nsplit > 1 ? (float *)(b + L.off_part) : nullptr;
  // calls of at most 32 query rows run one 32-query tile per workgroup
  const bool one_tile = t_q <= 32;
  const dim3 grid(one_tile ? 1u : (unsigned)(L.tq_pad / ATT_QB), (unsigned)n_head, (unsigned)nsplit);
  const int cz = causal ? 1 : 0;
  const int gw = cz | nsplit << 1 | n_head << 8;  // k_attn's packed grid
  if (rows && one_tile)
    hipLaunchKernelGGL((k_attn<true, 1>), grid, dim3(128), 0, s, (int)t_q, (int)t_kv, gw, (int)grid.x, q, (int)ldq, k,
                       (int)ldk, v, (int)ldv, out, (int)ldo, part, P, nullptr, 0, BeamCaches{});
  else if (rows)
    hipLaunchKernelGGL((k_attn<true, 2>), grid, dim3(128), 0, s, (int)t_q, (int)t_kv, gw, (int)grid.x, q, (int)ldq, k,
                       (int)ldk, v, (int)ldv, out, (int)ldo, part, P, nullptr, 0, BeamCaches{});
  else if (one_tile)
    hipLaunchKernelGGL((k_attn<false, 1>), grid, dim3(128), 0, s, (int)t_q, (int)t_kv, gw, (int)grid.x, q, (int)ldq,
                       nullptr, 0, nullptr, 0, out, (int)ldo, part, P, nullptr, 0, BeamCaches{});
  else
    hipLaunchKernelGGL((k_attn<false, 2>), grid, dim3(128), 0, s, (int)t_q, (int)t_kv, gw, (int)grid.x, q, (int)ldq,
                       nullptr, 0, nullptr, 0, out, (int)ldo, part, P, nullptr, 0, BeamCaches{});
  LAUNCH_TRY("k_attn");
  if (part) {
    const size_t nz = t_q * (size_t)n_head * ATT_DH;
    const bool with_rec = rec && t_q >= 2 && t_q <= (size_t)GEMV_MAX_M;
    hipLaunchKernelGGL(k_attn_combine, dim3((unsigned)cdiv(nz, 256)), dim3(256), 0, s, part, nsplit, n_head,
                       L.tq_pad, (int)t_q, out, (int)ldo, with_rec ? rec : nullptr, rec_off);
    LAUNCH_TRY("k_attn_combine");
    if (rec_done) *rec_done = with_rec;
  }
  return RW_OK;
}

// ------------------------------------------------------ decoder step

// Cross-attention K/V of every layer as the attention kernel's split planes,
// computed once per audio window and shared by forks.
struct CrossKV {
  int device = -1;
  size_t n_audio = 0, n = 0;
  int n_layer = 0, tkv_pad = 0;
  void *buf = nullptr;  // per layer: kh, kl, vh, vl planes of (n_head x 64) x tkv_pad f16
  size_t layer_bytes = 0, plane_bytes = 0;
  ~CrossKV() {
    if (buf) (void)hipFree(buf);
  }
  AttnPlanes planes(int l) const {
    const char *b = (const char *)buf + (size_t)l * layer_bytes;
    return AttnPlanes{nullptr, nullptr, (const uint16_t *)b, (const uint16_t *)(b + plane_bytes),
                      (const uint16_t *)(b + 2 * plane_bytes), (const uint16_t *)(b + 3 * plane_bytes), 0, tkv_pad};
  }
};

struct rw_decoder {
  rw_decoder_params p{};
  std::vector<rw_decoder_layer> layers;
  int device = -1;
  size_t n = 0, f = 0, n_audio = 0, n_past = 0;
  float *self_kv = nullptr;  // per layer: k then v, n_ctx x n each
  std::shared_ptr<CrossKV> cross;
  bool audio = false;
  void *scratch = nullptr;
  size_t scratch_cap = 0;
  ~rw_decoder() {
    if (self_kv) (void)hipFree(self_kv);
    if (scratch) (void)hipFree(scratch);
  }
  float *self_k(int l) const { return self_kv + (size_t)l * 2 * p.n_ctx * n; }
  float *self_v(int l) const { return self_kv + ((size_t)l * 2 + 1) * p.n_ctx * n; }
};

static int check_decoder_params(const rw_decoder_params *P) {
  if (!P || !P->layers || !P->token_embedding || !P->positional || !P->ln_w || !P->ln_b)
    return fail(RW_EINVAL, "decoder params, layers, token embedding, positional or final layernorm is NULL");
  if (P->n_layer <= 0 || P->n_ctx <= 0) return fail(RW_EINVAL, "n_layer and n_ctx must be positive");
  const size_t n = P->token_embedding->k;
  if (P->n_head <= 0 || n != (size_t)P->n_head * ATT_DH)
    return fail(RW_EINVAL, "n_state %zu != 64 * n_head (%d)", n, P->n_head);
  if (P->n_head >= (1 << 19)) return fail(RW_EINVAL, "n_head %d too large", P->n_head);
  const size_t f = P->layers[0].fc1 ? P->layers[0].fc1->n : 0;
  for (int l = 0; l < P->n_layer; ++l) {
    const rw_decoder_layer &L = P->layers[l];
    const rw_weight *sq[8] = {L.q, L.k, L.v, L.out, L.cq, L.ck, L.cv, L.cout};
    for (const rw_weight *w : sq)
      if (!w || w->n != n || w->k != n) return fail(RW_EINVAL, "layer %d: attention weights must be [%zu, %zu]", l, n, n);
    if (!L.fc1 || !L.fc2 || L.fc1->k != n || L.fc1->n != f || L.fc2->n != n || L.fc2->k != f)
      return fail(RW_EINVAL, "layer %d: fc1 must be [f, %zu] and fc2 [%zu, f]", l, n, n);
    const float *vec[6] = {L.attn_ln_w, L.attn_ln_b, L.cross_ln_w, L.cross_ln_b, L.mlp_ln_w, L.mlp_ln_b};
    for (const float *v : vec) {
      if (!v) return fail(RW_EINVAL, "layer %d: a layernorm vector is NULL", l);
      // the products that fold a layernorm in read it 16 bytes at a time
      if (!al16(v)) return fail(RW_EINVAL, "layer %d: layernorm vectors must be 16-byte aligned", l);
    }
  }
  if (!al16(P->ln_w) || !al16(P->ln_b)) return fail(RW_EINVAL, "the final layernorm vectors must be 16-byte aligned");
  return RW_OK;
}

// the per-call scratch of forward_hidden for n_tok tokens (beams: n_tok beams
// of one token each, whose self-attention runs as n_tok * n_head heads and
// whose new key / value rows pass through kn, vn)
struct DecScratch {
  size_t off_tok, off_x, off_cur, off_q, off_a, off_h, off_kn, off_vn, off_act, off_att, off_rec, bytes;
  AttnLayout self_att, cross_att;
};
static DecScratch dec_scratch(const rw_decoder *d, size_t n_tok, bool beams = false) {
  DecScratch S{};
  const size_t row = n_tok * d->n * 4;
  S.self_att = beams ? attn_layout(1, d->p.n_ctx, n_tok * d->n) : attn_layout(n_tok, d->p.n_ctx, d->n);
  S.cross_att = attn_layout(n_tok, d->n_audio, d->n, false);  // K/V: the window's kept planes
  S.off_tok = 0;
  S.off_x = align_up(n_tok * 4, 256);
  S.off_cur = align_up(S.off_x + row, 256);
  S.off_q = align_up(S.off_cur + row, 256);
  S.off_a = align_up(S.off_q + row, 256);
  S.off_h = align_up(S.off_a + row, 256);
  S.off_kn = align_up(S.off_h + n_tok * d->f * 4, 256);
  S.off_vn = align_up(S.off_kn + (beams ? row : 0), 256);
  S.off_act = align_up(S.off_vn + (beams ? row : 0), 256);
  S.off_att = align_up(S.off_act + act_layout(n_tok, std::max(d->n, d->f)).bytes, 256);
  S.off_rec = align_up(S.off_att + std::max(S.self_att.bytes, S.cross_att.bytes), 256);
  // activation records passed between products (decode sizes): fc2's from
  // fc1, cross-out's from the cross-attention's merge
  const size_t rec =
      n_tok <= (size_t)GEMV_MAX_M ? align_up(std::max(d->f, d->n), 256) / QK * gemv_rec_bytes((int)n_tok) : 0;
  S.bytes = align_up(S.off_rec + rec, 256);
  return S;
}

// One self-attention over several beams' caches (one new row each): the
// planes of beam b, head h are head b * n_head + h of one k_attn launch.
// rec: without a kv split, k_attn also writes the output rows' activation
// records for the next product (offset term rec_off); *rec_done says
// whether it did.
static int run_beam_self_attention(rw_decoder *const *beams, size_t nb, int l, const float *q, const float *kn,
                                   const float *vn, float *att, const AttnLayout &L, void *ws, hipStream_t s,
                                   uint8_t *rec = nullptr, int rec_off = 0, bool *rec_done = nullptr) {
  if (rec_done) *rec_done = false;
  const rw_decoder *d = beams[0];
  const int n_head = d->p.n_head, heads = (int)nb * n_head;
  const size_t n_past = d->n_past, t_kv = n_past + 1;
  char *b = (char *)ws;
  AttnPlanes P{(uint16_t *)(b + L.off_qh), (uint16_t *)(b + L.off_ql), (uint16_t *)(b + L.off_kh),
               (uint16_t *)(b + L.off_kl), (uint16_t *)(b + L.off_vh), (uint16_t *)(b + L.off_vl), L.tq_pad,
               (int)std::min<size_t>(align_up(t_kv, ATT_KVB), L.tkv_pad)};
  BeamCaches C{};
  for (size_t i = 0; i < nb; ++i) {
    C.k[i] = beams[i]->self_k(l);
    C.v[i] = beams[i]->self_v(l);
  }
  // one launch: each (beam, head) plane splits its q row and its beam's
  // cached K and V rows as it loads them, takes the newest row from kn / vn
  // and stores it into the beam's caches
  const int nsplit = std::min(L.nsplit, attn_nsplit((size_t)(L.tq_pad / ATT_QB) * heads, cdiv(t_kv, ATT_KVB)));
  float *part = nsplit > 1 ? (float *)(b + L.off_part) : nullptr;
  const bool with_rec = rec && !part && nb >= 2 && nb <= (size_t)GEMV_MAX_M;
  hipLaunchKernelGGL((k_attn<true, 1, true>), dim3(1, (unsigned)heads, (unsigned)nsplit), dim3(128), 0, s, 1,
                     (int)t_kv, 1 | nsplit << 1 | heads << 8, 1, q, (int)d->n, kn, (int)d->n, vn, (int)d->n, att,
                     (int)d->n, part, P, with_rec ? rec : nullptr, n_head | rec_off << 8 | (int)nb << 16, C);
  LAUNCH_TRY("k_attn");
  if (rec_done) *rec_done = with_rec;
  if (part) {
    hipLaunchKernelGGL(k_attn_combine, dim3((unsigned)cdiv((size_t)heads * ATT_DH, 256)), dim3(256), 0, s, part, nsplit,
                       heads, L.tq_pad, 1, att, (int)d->n, nullptr, 0);
    LAUNCH_TRY("k_attn_combine");
  }
  return RW_OK;
}

// y = layernorm(x (+= r first when r is given))
static int launch_layernorm(float *x, size_t rows, size_t n, const float *w, const float *b, float *y,
                            hipStream_t s, const float *r) {
  hipLaunchKernelGGL(k_layernorm, dim3((unsigned)rows), dim3(256), 0, s, x, (int)n, w, b, y, r);
  LAUNCH_TRY("k_layernorm");
  return RW_OK;
}

// One forward pass: n_tok tokens of one decoder (nb = 1, beams = false), or
// one token for each of nb beams (forks sharing the cross K/V at one n_past,
// n_tok = nb, beams = true).
static int decoder_forward(rw_decoder *const *dec, size_t nb, bool beams, size_t n_tok, float *hidden, char *b,
                           const DecScratch &S, hipStream_t s) {
  rw_decoder *d = dec[0];
  const size_t n = d->n;
  const int *tok = (const int *)(b + S.off_tok);
  float *x = (float *)(b + S.off_x), *cur = (float *)(b + S.off_cur), *q = (float *)(b + S.off_q);
  float *att = (float *)(b + S.off_a), *h = (float *)(b + S.off_h);
  float *kn = (float *)(b + S.off_kn), *vn = (float *)(b + S.off_vn);
  void *act = b + S.off_act, *aws = b + S.off_att;
  const rw_weight *E = d->p.token_embedding;
  const size_t items = n_tok * (size_t)E->nb;
#define RW_EMB(DT)                                                                                           \
  hipLaunchKernelGGL(k_embed<DT>, dim3((unsigned)cdiv(items, 256)), dim3(256), 0, s, E->view, tok, (int)n_tok, \
                     d->p.positional, (int)d->n_past, beams ? 0 : 1, x)
  switch (E->dtype) {
    case RW_Q4_0: RW_EMB(RW_Q4_0); break;
    case RW_Q4_1: RW_EMB(RW_Q4_1); break;
    case RW_Q5_0: RW_EMB(RW_Q5_0); break;
    case RW_Q5_1: RW_EMB(RW_Q5_1); break;
    default: RW_EMB(RW_Q8_0); break;
  }
#undef RW_EMB
  LAUNCH_TRY("k_embed");
  const size_t t_kv = d->n_past + n_tok;
  // x is the residual stream: every layernorm is folded into the product
  // that reads it, and every residual add (src/decoder.rs:168-170, 191-193,
  // mlp_block) into the epilogue of the product that makes it
  for (int l = 0; l < d->p.n_layer; ++l) {
    const rw_decoder_layer &L = d->layers[l];
    // causal self-attention over the cache and the new rows
    {
      // q, k and v in one launch; k and v land in the cache rows (beams: in
      // kn, vn, which the beams' split stores into each beam's cache)
      const rw_weight *w3[3] = {L.q, L.k, L.v};
      const float *b3[3] = {L.q_b, nullptr, L.v_b};
      float *o3[3] = {q, beams ? kn : d->self_k(l) + d->n_past * n, beams ? vn : d->self_v(l) + d->n_past * n};
      if (L.q->dtype == L.k->dtype && L.q->dtype == L.v->dtype) {
        RW_TRY(run_matmul_set(w3, 3, x, n_tok, b3, o3, act, s, L.attn_ln_w, L.attn_ln_b, 0, cur));
      } else {
        RW_TRY(launch_layernorm(x, n_tok, n, L.attn_ln_w, L.attn_ln_b, cur, s, nullptr));
        for (int i = 0; i < 3; ++i) RW_TRY(run_matmul(w3[i], cur, n_tok, b3[i], o3[i], act, s));
      }
    }
    // several beams: where their self-attention runs unsplit it also writes
    // out's activation records (whole octets of blocks), which out copies
    uint8_t *orec = n_tok >= 2 && n_tok <= (size_t)GEMV_MAX_M && n % (OCT * QK) == 0 ? (uint8_t *)(b + S.off_rec)
                                                                                     : nullptr;
    bool orec_done = false;
    const int ooff = L.out->dtype == RW_Q4_0 ? 8 : L.out->dtype == RW_Q5_0 ? 16 : 0;
    if (beams)
      RW_TRY(run_beam_self_attention(dec, nb, l, q, kn, vn, att, S.self_att, aws, s, orec, ooff, &orec_done));
    else
      RW_TRY(run_attention(q, n, d->self_k(l), n, d->self_v(l), n, n_tok, t_kv, d->p.n_head, 1, att, n, S.self_att,
                           aws, s));
    RW_TRY(run_linear(L.out, att, n_tok, L.out_b, x, act, s, nullptr, nullptr, GEMM_ACC, nullptr, nullptr,
                      orec_done ? orec : nullptr));
    // cross-attention to the window's K/V
    RW_TRY(run_linear(L.cq, x, n_tok, L.cq_b, q, act, s, L.cross_ln_w, L.cross_ln_b, 0, cur));
    const AttnPlanes cp = d->cross->planes(l);
    // for 2-8 rows the merge of the split kv also writes cross-out's
    // activation records (whole octets of blocks), which cross-out copies
    uint8_t *crec = n_tok >= 2 && n_tok <= (size_t)GEMV_MAX_M && n % (OCT * QK) == 0 ? (uint8_t *)(b + S.off_rec)
                                                                                     : nullptr;
    bool crec_done = false;
    const int coff = L.cout->dtype == RW_Q4_0 ? 8 : L.cout->dtype == RW_Q5_0 ? 16 : 0;
    RW_TRY(run_attention(q, n, nullptr, n, nullptr, n, n_tok, d->n_audio, d->p.n_head, 0, att, n, S.cross_att, aws,
                         s, &cp, crec, coff, &crec_done));
    RW_TRY(run_linear(L.cout, att, n_tok, L.cout_b, x, act, s, nullptr, nullptr, GEMM_ACC, nullptr, nullptr,
                      crec_done ? crec : nullptr));
    // MLP.  For 2-8 rows fc1's epilogue also writes fc2's activation records
    // (the values fc2 would quantize in each of its workgroups; whole octets
    // of blocks, one dtype), and fc2 copies them: the 5-beam step 3.42 ->
    // 3.21 ms, the same bits.  One row keeps fc2's fill from the values it
    // loads into registers (2.03 against 2.05 ms per token with records)
    uint8_t *rec = n_tok >= 2 && n_tok <= (size_t)GEMV_MAX_M && L.fc1->n % (OCT * QK) == 0 &&
                           L.fc1->dtype == L.fc2->dtype
                       ? (uint8_t *)(b + S.off_rec)
                       : nullptr;
    RW_TRY(run_linear(L.fc1, x, n_tok, L.fc1_b, h, act, s, L.mlp_ln_w, L.mlp_ln_b, GEMM_GELU, cur, rec));
    RW_TRY(run_linear(L.fc2, h, n_tok, L.fc2_b, x, act, s, nullptr, nullptr, GEMM_ACC, nullptr, nullptr, rec));
  }
  return launch_layernorm(x, n_tok, n, d->p.ln_w, d->p.ln_b, hidden, s, nullptr);
}

// ------------------------------------------------------ encoder layer

struct LayerLayout {
  size_t n, f;
  ActLayout act;  // the quantized activation of the widest product (fc2's)
  AttnLayout att;
  size_t off_act, off_q, off_k, off_v, off_a, off_h, off_att, bytes;
};

static LayerLayout layer_layout(size_t n, size_t f, size_t t) {
  LayerLayout L{};
  L.n = n;
  L.f = f;
  L.act = act_layout(t, std::max(n, f));
  L.att = attn_layout(t, t, n);
  const size_t row = t * n * 4;
  L.off_act = 0;
  L.off_q = align_up(L.act.bytes, 256);
  L.off_k = align_up(L.off_q + row, 256);
  L.off_v = align_up(L.off_k + row, 256);
  L.off_a = align_up(L.off_v + row, 256);
  L.off_h = align_up(L.off_a + row, 256);
  L.off_att = align_up(L.off_h + std::max(t * f * 4, fused_quant_bytes(t, f)), 256);
  L.bytes = align_up(L.off_att + L.att.bytes, 256);
  return L;
}


static int check_layer(const rw_encoder_layer *E, size_t t) {
  if (!E) return fail(RW_EINVAL, "layer is NULL");
  if (!E->q || !E->k || !E->v || !E->out || !E->fc1 || !E->fc2) return fail(RW_EINVAL, "a layer weight is NULL");
  if (!E->attn_ln_w || !E->attn_ln_b || !E->mlp_ln_w || !E->mlp_ln_b)
    return fail(RW_EINVAL, "a layernorm vector is NULL");
  const size_t n = E->q->k, f = E->fc1->n;
  if (E->n_head <= 0 || n != (size_t)E->n_head * ATT_DH)
    return fail(RW_EINVAL, "n_state %zu != 64 * n_head (%d)", n, E->n_head);
  const rw_weight *sq[4] = {E->q, E->k, E->v, E->out};
  for (const rw_weight *w : sq)
    if (w->n != n || w->k != n || w->dtype != E->q->dtype)
      return fail(RW_EINVAL, "q, k, v and out must be [%zu, %zu] of one dtype", n, n);
  if (E->fc1->k != n || E->fc2->n != n || E->fc2->k != f)
    return fail(RW_EINVAL, "fc1 must be [f, %zu] and fc2 [%zu, f] (f = %zu)", n, n, f);
  if (t <= (size_t)GEMV_MAX_M) return fail(RW_EINVAL, "t = %zu: the layer takes more than %d rows", t, GEMV_MAX_M);
  if (t > (1u << 20)) return fail(RW_EINVAL, "t = %zu is too large", t);
  if (!al16(E->attn_ln_w) || !al16(E->attn_ln_b) || !al16(E->mlp_ln_w) || !al16(E->mlp_ln_b))
    return fail(RW_EINVAL, "layernorm vectors must be 16-byte aligned");
  return RW_OK;
}

static int run_encoder_layer(const rw_encoder_layer *E, float *x, size_t t, void *ws, hipStream_t s) {
  const LayerLayout L = layer_layout(E->q->k, E->fc1->n, t);
  char *b = (char *)ws;
  float *qb = (float *)(b + L.off_q), *kb = (float *)(b + L.off_k), *vb = (float *)(b + L.off_v);
  float *ab = (float *)(b + L.off_a), *hb = (float *)(b + L.off_h);
  const size_t n = L.n, f = L.f;
  const ActLayout Ln = act_layout(t, n), Lf = act_layout(t, f);
  const int m = (int)t;
  // x + out(attn(q, k, v of ln1(x)))
  int rc = launch_quantize(x, t, n, Ln, b, s, E->attn_ln_w, E->attn_ln_b);
  if (rc) return rc;
  {
    const rw_weight *w3[3] = {E->q, E->k, E->v};
    const float *b3[3] = {E->q_b, E->k_b, E->v_b};
    float *o3[3] = {qb, kb, vb};
    rc = run_gemm(w3, b3, o3, 3, act_view(Ln, b), m, s);
    if (rc) return rc;
  }
  rc = run_attention(qb, n, kb, n, vb, n, t, t, E->n_head, 0, ab, n, L.att, b + L.off_att, s);
  if (rc) return rc;
  rc = launch_quantize(ab, t, n, Ln, b, s);
  if (rc) return rc;
  const int acc = GEMM_ACC, act = GEMM_GELU;
  rc = run_gemm(&E->out, &E->out_b, &x, 1, act_view(Ln, b), m, s, &acc);
  if (rc) return rc;
  // x + fc2(gelu(fc1(ln2(x))))
  rc = launch_quantize(x, t, n, Ln, b, s, E->mlp_ln_w, E->mlp_ln_b);
  if (rc) return rc;
  // fc2's activation: by default fc1 writes gelu(y) in f32 and a quantize
  // launch reads it back; RW_ENCODER_MLP=fused quantizes it in fc1's epilogue
  // instead (int8 quants and block maxima in h's space, then the f16 plane:
  // bitwise the same operand; measured 1-2 us per large-v3 layer slower, the
  // epilogue's quantization costing more than the f32 round trip it saves)
  const char *mlp = getenv("RW_ENCODER_MLP");
  if (f % QK == 0 && mlp && !strcmp(mlp, "fused")) {
    int8_t *qh = (int8_t *)hb;  // [row group][block][32][32], then the block maxima
    float *ah = (float *)(b + L.off_h + align_up(cdiv(t, RG) * RG * f, 256));
    const int fq = GEMM_GELU | GEMM_QUANT;
    rc = run_gemm(&E->fc1, &E->fc1_b, &hb, 1, act_view(Ln, b), m, s, &fq, qh, ah);
    if (rc) return rc;
    rc = launch_quantize_finish(qh, ah, t, f, Lf, b, s);
  } else {
    rc = run_gemm(&E->fc1, &E->fc1_b, &hb, 1, act_view(Ln, b), m, s, &act);
    if (rc) return rc;
    rc = launch_quantize(hb, t, f, Lf, b, s);
  }
  if (rc) return rc;
  return run_gemm(&E->fc2, &E->fc2_b, &x, 1, act_view(Lf, b), m, s, &acc);
}

extern "C" {

int rw_rocm_version(void) { return 0x000100; }

int rw_rocm_last_error(char *buf, size_t len) {
  if (buf && len) {
    size_t c = g_err.size() < len - 1 ? g_err.size() : len - 1;
    memcpy(buf, g_err.data(), c);
    buf[c] = 0;
  }
  return (int)g_err.size();
}

int rw_rocm_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  int ok = 0;
  for (int d = 0; d < n; ++d)
    if (check_device(d) == RW_OK) ++ok;
  return ok;
}

int rw_rocm_init(int device) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
    (void)hipGetLastError();
    return fail(RW_ENODEV, "no HIP device visible");
  }
  if (device < 0 || device >= n) return fail(RW_ENODEV, "device %d out of range (%d visible)", device, n);
  int rc = check_device(device);
  if (rc) return rc;
  HIP_TRY(hipSetDevice(device));
  return scratch_setup(device, nullptr);
}

int rw_rocm_block_bytes(int dtype) {
  int bb = bb_of(dtype);
  return bb < 0 ? fail(RW_EINVAL, "unsupported dtype %d", dtype) : bb;
}

int rw_rocm_weight_upload(int dtype, size_t n, size_t k, const uint8_t *raw, size_t raw_len, rw_weight **out) {
  if (!out) return fail(RW_EINVAL, "out is NULL");
  *out = nullptr;
  int bb = bb_of(dtype);
  if (bb < 0) return fail(RW_EINVAL, "unsupported dtype %d", dtype);
  if (k == 0 || k % QK) return fail(RW_EINVAL, "k must be a positive multiple of %d (got %zu)", QK, k);
  if (n == 0) return fail(RW_EINVAL, "n must be positive");
  if (k / QK > (size_t)1 << 24 || n > (size_t)1 << 28) return fail(RW_EINVAL, "shape [%zu, %zu] too large", n, k);
  size_t nb = k / QK;
  if (raw_len != n * nb * (size_t)bb)
    return fail(RW_EINVAL, "raw length %zu != n*(k/32)*block_bytes = %zu", raw_len, n * nb * (size_t)bb);
  if (!raw) return fail(RW_EINVAL, "raw is NULL");
  int dev;
  int rc = current_device(&dev);
  if (rc) return rc;

  rw_weight *w = new rw_weight();
  w->dtype = dtype;
  w->device = dev;
  w->n = n;
  w->k = k;
  w->nb = (int)nb;
  w->nb_pad = (int)align_up(nb, OCT);
  w->noct = w->nb_pad / OCT;
  w->ngroups = (int)cdiv(n, RG);
  size_t rows = (size_t)w->ngroups * RG;
  size_t nsc = rows * w->nb_pad;
  size_t qsz = nsc * qs_bytes(dtype);
  size_t off_qh = align_up(qsz, 256);
  size_t off_d = align_up(off_qh + (has_high(dtype) ? nsc * 4 : 0), 256);
  size_t off_m = align_up(off_d + nsc * 2, 256);
  size_t off_dm = align_up(off_m + (has_min(dtype) ? nsc * 2 : 0), 256);
  size_t off_q8 = align_up(off_dm + nsc * 4, 256);  // the GEMM's byte plane (Q8_0 reads qs)
  size_t off_cs = align_up(off_q8 + (dtype == RW_Q8_0 ? 0 : nsc * 32), 256);  // the GEMM's row scales
  size_t off_cm = align_up(off_cs + rows * 4, 256);                             // and row offsets
  w->bytes = align_up(off_cm + rows * 4, 256);
  // the kernels address each plane with 32-bit byte offsets
  if (nsc * 32 >= ((size_t)1 << 32)) {
    delete w;
    return fail(RW_EINVAL, "shape [%zu, %zu]: a resident plane would exceed 4 GiB", n, k);
  }
  if (hipMalloc(&w->base, w->bytes) != hipSuccess) {
    (void)hipGetLastError();
    delete w;
    return fail(RW_ENOMEM, "hipMalloc(%zu) for a [%zu, %zu] weight failed", w->bytes, n, k);
  }
  char *b = (char *)w->base;
  w->view = WeightView{(const uint8_t *)b, (const uint32_t *)(b + off_qh), (const uint16_t *)(b + off_d),
                       (const uint16_t *)(b + off_m), w->nb, w->nb_pad, w->noct, w->ngroups};
  w->gemm = GemmPlanes{(const uint8_t *)(dtype == RW_Q8_0 ? b : b + off_q8), (const uint32_t *)(b + off_dm),
                       (const float *)(b + off_cs), (const float *)(b + off_cm)};

  void *tmp = nullptr;
  hipError_t e = hipMalloc(&tmp, raw_len);
  if (e == hipSuccess) e = hipMemcpy(tmp, raw, raw_len, hipMemcpyHostToDevice);
  if (e == hipSuccess) {
    size_t threads = nsc;
    dim3 grid((unsigned)cdiv(threads, 256));
    // the GEMM's row scales first (one wavefront per row), then the planes
#define RW_REPACK(DT)                                                                                      \
  hipLaunchKernelGGL(k_row_scale<DT>, dim3((unsigned)cdiv(rows, 4)), dim3(256), 0, 0, (const uint8_t *)tmp,   \
                     (int)n, (int)nb, (int)rows, (float *)(b + off_cs), (float *)(b + off_cm));           \
  hipLaunchKernelGGL(k_repack<DT>, grid, dim3(256), 0, 0, (const uint8_t *)tmp, (int)n, (int)nb, (uint8_t *)b, \
                     (uint32_t *)(b + off_qh), (uint16_t *)(b + off_d), (uint16_t *)(b + off_m),                \
                     (uint32_t *)(b + off_dm), (uint8_t *)(b + off_q8), w->nb_pad,                        \
                     w->noct, w->ngroups, (const float *)(b + off_cs), (const float *)(b + off_cm))
    switch (dtype) {
      case RW_Q4_0: RW_REPACK(RW_Q4_0); break;
      case RW_Q4_1: RW_REPACK(RW_Q4_1); break;
      case RW_Q5_0: RW_REPACK(RW_Q5_0); break;
      case RW_Q5_1: RW_REPACK(RW_Q5_1); break;
      default: RW_REPACK(RW_Q8_0); break;
    }
#undef RW_REPACK
    e = hipGetLastError();
    if (e == hipSuccess) e = hipStreamSynchronize(nullptr);
    if (e == hipSuccess) {
      // a weight with no offset row skips the offset term in the GEMM
      std::vector<float> cm(rows);
      e = hipMemcpy(cm.data(), b + off_cm, rows * 4, hipMemcpyDeviceToHost);
      bool any = false;
      for (float v : cm) any = any || v != 0.0f;
      if (!any) w->gemm.cm = nullptr;
    }
  }
  if (tmp) (void)hipFree(tmp);
  if (e != hipSuccess) {
    (void)hipFree(w->base);
    delete w;
    return fail(RW_EHIP, "weight upload: %s", hipGetErrorString(e));
  }
  *out = w;
  return RW_OK;
}

int rw_rocm_weight_free(rw_weight *w) {
  if (!w) return RW_OK;
  int prev = -1;
  (void)hipGetDevice(&prev);
  (void)hipSetDevice(w->device);
  hipError_t e = hipFree(w->base);
  if (prev >= 0) (void)hipSetDevice(prev);
  delete w;
  if (e != hipSuccess) return fail(RW_EHIP, "hipFree: %s", hipGetErrorString(e));
  return RW_OK;
}

int rw_rocm_weight_info(const rw_weight *w, int *dtype, size_t *n, size_t *k, size_t *device_bytes) {
  if (!w) return fail(RW_EINVAL, "weight is NULL");
  if (dtype) *dtype = w->dtype;
  if (n) *n = w->n;
  if (k) *k = w->k;
  if (device_bytes) *device_bytes = w->bytes;
  return RW_OK;
}

size_t rw_rocm_matmul_workspace_size(size_t m, size_t k) {
  if (k == 0 || k % QK || m == 0) return 0;
  return act_layout(m, k).bytes;
}

int rw_rocm_matmul_t_q_dev(const rw_weight *w, const float *a, size_t m, size_t k, const float *bias, float *out,
                           void *workspace, size_t workspace_len, void *stream) {
  int rc = check_matmul_args(w, a, m, k, out);
  if (rc) return rc;
  if (m == 0) return RW_OK;
  HIP_TRY(hipSetDevice(w->device));
  size_t need = act_layout(m, k).bytes;
  void *ws = workspace;
  WsHold hold;  // the stream's workspace, held until the launches are queued
  if (m <= GEMV_MAX_M) {
    ws = nullptr;  // the decode shape quantizes inside its launch
  } else if (ws) {
    if (workspace_len < need) return fail(RW_EINVAL, "workspace of %zu bytes < %zu needed", workspace_len, need);
  } else {
    rc = stream_workspace(w->device, stream, need, hold, &ws);
    if (rc) return rc;
  }
  return run_matmul(w, a, m, bias, out, ws, (hipStream_t)stream);
}

int rw_rocm_matmul_t_q_dev_noalloc(const rw_weight *w, const float *a, size_t m, size_t k, const float *bias,
                                   float *out, void *stream) {
  int rc = check_matmul_args(w, a, m, k, out);
  if (rc) return rc;
  if (m == 0) return RW_OK;
  const size_t need = m <= GEMV_MAX_M ? 0 : act_layout(m, k).bytes;  // the decode shape needs none
  if (need > (size_t)RW_NOALLOC_SCRATCH_BYTES)
    return fail(RW_EINVAL, "[%zu, %zu] activation needs %zu workspace bytes, more than the %d of the fixed scratch", m,
                k, need, RW_NOALLOC_SCRATCH_BYTES);
  HIP_TRY(hipSetDevice(w->device));
  void *ws = nullptr;
  rc = scratch_setup(w->device, &ws);
  if (rc) return rc;
  // every byte the product reads is written by its quantizer first (padding
  // rows included), so nothing needs clearing between calls
  return run_matmul(w, a, m, bias, out, m <= GEMV_MAX_M ? nullptr : ws, (hipStream_t)stream);
}

int rw_rocm_quantize_dev(const float *a, size_t m, size_t k, void *workspace, size_t workspace_len,
                         void *stream) {
  if (k == 0 || k % QK) return fail(RW_EINVAL, "k must be a positive multiple of %d (got %zu)", QK, k);
  if (m == 0) return RW_OK;
  if (!a || !workspace) return fail(RW_EINVAL, "activation or workspace pointer is NULL");
  if (m > (size_t)INT32_MAX / 2) return fail(RW_EINVAL, "m = %zu is too large", m);
  ActLayout L = act_layout(m, k);
  if (workspace_len < L.bytes) return fail(RW_EINVAL, "workspace of %zu bytes < %zu needed", workspace_len, L.bytes);
  return launch_quantize(a, m, k, L, workspace, (hipStream_t)stream);
}

int rw_rocm_matmul_prequant_dev(const rw_weight *w, const void *workspace, size_t m, const float *bias,
                                float *out, void *stream) {
  if (!w) return fail(RW_EINVAL, "weight is NULL");
  if (m == 0) return RW_OK;
  if (!workspace || !out) return fail(RW_EINVAL, "workspace or output pointer is NULL");
  if (m > (size_t)INT32_MAX / 2) return fail(RW_EINVAL, "m = %zu is too large", m);
  HIP_TRY(hipSetDevice(w->device));
  return run_product(w, m, bias, out, workspace, (hipStream_t)stream);
}

int rw_rocm_matmul_prequant_multi_dev(const rw_weight *const *w, size_t count, const void *workspace, size_t m,
                                      const float *const *bias, float *const *out, void *stream) {
  if (!w || !out) return fail(RW_EINVAL, "weight or output array is NULL");
  if (count < 1 || count > (size_t)GEMM_MAX_SET)
    return fail(RW_EINVAL, "count = %zu: between 1 and %d weights per call", count, GEMM_MAX_SET);
  for (size_t i = 0; i < count; ++i) {
    if (!w[i] || !out[i]) return fail(RW_EINVAL, "weight or output %zu is NULL", i);
    if (w[i]->dtype != w[0]->dtype || w[i]->k != w[0]->k || w[i]->device != w[0]->device)
      return fail(RW_EINVAL, "weight %zu differs from weight 0 in dtype, k or device", i);
  }
  if (m == 0) return RW_OK;
  if (!workspace) return fail(RW_EINVAL, "workspace is NULL");
  if (m > (size_t)INT32_MAX / 2) return fail(RW_EINVAL, "m = %zu is too large", m);
  HIP_TRY(hipSetDevice(w[0]->device));
  hipStream_t s = (hipStream_t)stream;
  if (m <= GEMV_MAX_M) {  // the decode shape: one GEMV launch per weight
    for (size_t i = 0; i < count; ++i) {
      int rc = run_product(w[i], m, bias ? bias[i] : nullptr, out[i], workspace, s);
      if (rc) return rc;
    }
    return RW_OK;
  }
  ActLayout L = act_layout(m, w[0]->k);
  return run_gemm(w, bias, out, count, act_view(L, (void *)workspace), (int)m, s);
}

size_t rw_rocm_gelu_quantize_workspace_size(size_t m, size_t n) {
  if (m <= (size_t)GEMV_MAX_M || n == 0 || n % QK) return 0;
  return align_up(act_layout(m, n).bytes, 256) + fused_quant_bytes(m, n);
}

int rw_rocm_matmul_prequant_gelu_quantize_dev(const rw_weight *w, const void *workspace, size_t m,
                                              const float *bias, void *next_workspace, size_t next_len,
                                              void *stream) {
  if (!w) return fail(RW_EINVAL, "weight is NULL");
  if (m == 0) return RW_OK;
  if (!workspace || !next_workspace) return fail(RW_EINVAL, "workspace pointer is NULL");
  if (m <= (size_t)GEMV_MAX_M)
    return fail(RW_EINVAL, "m = %zu: the fused GELU + quantization takes more than %d rows", m, GEMV_MAX_M);
  if (m > (size_t)INT32_MAX / 2) return fail(RW_EINVAL, "m = %zu is too large", m);
  if (w->n % QK) return fail(RW_EINVAL, "n = %zu must be a multiple of %d (the next product's k)", w->n, QK);
  const size_t need = rw_rocm_gelu_quantize_workspace_size(m, w->n);
  if (next_len < need) return fail(RW_EINVAL, "next workspace of %zu bytes < %zu needed", next_len, need);
  HIP_TRY(hipSetDevice(w->device));
  hipStream_t s = (hipStream_t)stream;
  const ActLayout Lin = act_layout(m, w->k), Lout = act_layout(m, w->n);
  char *nx = (char *)next_workspace;
  int8_t *q = (int8_t *)(nx + align_up(Lout.bytes, 256));
  float *am = (float *)(nx + align_up(Lout.bytes, 256) + align_up(cdiv(m, RG) * RG * w->n, 256));
  const int fq = GEMM_GELU | GEMM_QUANT;
  float *none = nullptr;  // no f32 output in this mode
  int rc = run_gemm(&w, &bias, &none, 1, act_view(Lin, (void *)workspace), (int)m, s, &fq, q, am);
  if (rc) return rc;
  return launch_quantize_finish(q, am, m, w->n, Lout, next_workspace, s);
}

int rw_rocm_matmul_t_q(const rw_weight *w, const float *a, size_t m, size_t k, const float *bias, float *out) {
  int rc = check_matmul_args(w, a, m, k, out);
  if (rc) return rc;
  if (m == 0) return RW_OK;
  HIP_TRY(hipSetDevice(w->device));
  CtxGuard g;
  rc = ctx_acquire(w->device, &g.c);
  if (rc) return rc;
  Ctx *c = g.c;
  ActLayout L = act_layout(m, k);
  size_t off_a = align_up(L.bytes, 256);
  size_t off_o = align_up(off_a + m * k * 4, 256);
  size_t off_b = align_up(off_o + m * w->n * 4, 256);
  size_t total = align_up(off_b + w->n * 4, 256);
  rc = ctx_reserve(c, total);
  if (rc) return rc;
  char *b = (char *)c->buf;
  float *da = (float *)(b + off_a), *dout = (float *)(b + off_o), *dbias = bias ? (float *)(b + off_b) : nullptr;
  HIP_TRY(hipMemcpyAsync(da, a, m * k * 4, hipMemcpyHostToDevice, c->stream));
  if (bias) HIP_TRY(hipMemcpyAsync(dbias, bias, w->n * 4, hipMemcpyHostToDevice, c->stream));
  rc = run_matmul(w, da, m, dbias, dout, b, c->stream);
  if (rc) {
    (void)hipStreamSynchronize(c->stream);
    return rc;
  }
  HIP_TRY(hipMemcpyAsync(out, dout, m * w->n * 4, hipMemcpyDeviceToHost, c->stream));
  HIP_TRY(hipStreamSynchronize(c->stream));
  return RW_OK;
}

// ------------------------------------------------------ dense f32 tier

static int check_dense_args(const float *a, size_t m, size_t k, const float *b, size_t n, const float *out) {
  if (m && (!a || !out)) return fail(RW_EINVAL, "a or out is NULL");
  if (!b) return fail(RW_EINVAL, "b is NULL");
  if (k == 0 || n == 0) return fail(RW_EINVAL, "k and n must be positive");
  // grid: n / 32 tiles along x, m / 32 along y (at most 65535)
  if (cdiv(m, 32) > 65535 || n > ((size_t)1 << 31) - 32 || k > ((size_t)1 << 31) - 1)
    return fail(RW_EINVAL, "shape [%zu, %zu] x [%zu, %zu]^T too large", m, k, n, k);
  return RW_OK;
}

static int launch_matmul_t_f32(const float *a, size_t m, size_t k, const float *b, size_t n, const float *bias,
                               float *out, hipStream_t s) {
  hipLaunchKernelGGL(k_matmul_t_f32, dim3((unsigned)cdiv(n, 32), (unsigned)cdiv(m, 32)), dim3(256), 0, s, a, b, bias,
                     out, (int)m, (int)n, (int)k);
  LAUNCH_TRY("k_matmul_t_f32");
  return RW_OK;
}

int rw_rocm_matmul_t_f32_dev(const float *a, size_t m, size_t k, const float *b, size_t n, const float *bias,
                             float *out, void *stream) {
  int rc = check_dense_args(a, m, k, b, n, out);
  if (rc || m == 0) return rc;
  return launch_matmul_t_f32(a, m, k, b, n, bias, out, (hipStream_t)stream);
}

int rw_rocm_matmul_t_f32(const float *a, size_t m, size_t k, const float *b, size_t n, const float *bias,
                         float *out) {
  int rc = check_dense_args(a, m, k, b, n, out);
  if (rc || m == 0) return rc;
  int dev;
  HIP_TRY(hipGetDevice(&dev));
  rc = check_device(dev);
  if (rc) return rc;
  CtxGuard g;
  rc = ctx_acquire(dev, &g.c);
  if (rc) return rc;
  Ctx *c = g.c;
  const size_t off_b = align_up(m * k * 4, 256), off_o = align_up(off_b + n * k * 4, 256);
  const size_t off_bias = align_up(off_o + m * n * 4, 256), total = align_up(off_bias + n * 4, 256);
  rc = ctx_reserve(c, total);
  if (rc) return rc;
  char *buf = (char *)c->buf;
  float *da = (float *)buf, *db = (float *)(buf + off_b), *dout = (float *)(buf + off_o);
  float *dbias = bias ? (float *)(buf + off_bias) : nullptr;
  HIP_TRY(hipMemcpyAsync(da, a, m * k * 4, hipMemcpyHostToDevice, c->stream));
  HIP_TRY(hipMemcpyAsync(db, b, n * k * 4, hipMemcpyHostToDevice, c->stream));
  if (bias) HIP_TRY(hipMemcpyAsync(dbias, bias, n * 4, hipMemcpyHostToDevice, c->stream));
  rc = launch_matmul_t_f32(da, m, k, db, n, dbias, dout, c->stream);
  if (rc) {
    (void)hipStreamSynchronize(c->stream);
    return rc;
  }
  HIP_TRY(hipMemcpyAsync(out, dout, m * n * 4, hipMemcpyDeviceToHost, c->stream));
  HIP_TRY(hipStreamSynchronize(c->stream));
  return RW_OK;
}

size_t rw_rocm_grouped_workspace_size(const rw_linear *items, size_t count) {
  if (!items) return 0;
  return group_plan(items, count).total;
}

int rw_rocm_matmul_grouped_dev(const rw_linear *items, size_t count, void *workspace, size_t workspace_len,
                               void *stream) {
  if (count == 0) return RW_OK;
  if (!items) return fail(RW_EINVAL, "items is NULL");
  int rc0 = check_group_items(items, count);
  if (rc0) return rc0;
  GroupPlan P = group_plan(items, count);
  if (P.order.empty()) return RW_OK;
  const int device = items[0].w->device;
  HIP_TRY(hipSetDevice(device));
  void *ws = workspace;
  WsHold hold;
  if (ws) {
    if (workspace_len < P.total) return fail(RW_EINVAL, "workspace of %zu bytes < %zu needed", workspace_len, P.total);
  } else {
    int rc = stream_workspace(device, stream, P.total, hold, &ws);
    if (rc) return rc;
  }
  hipStream_t s = (hipStream_t)stream;
  {
    // the tables go up through pinned memory of this (device, stream); the
    // previous copy out of it must have finished before it is rewritten
    std::lock_guard<std::mutex> lk(g_stage_mu);
    Stage &st = g_stage[std::make_pair(device, stream)];
    if (st.pending) {
      HIP_TRY(hipEventSynchronize(st.ev));
      st.pending = false;
    }
    if (!st.ev) HIP_TRY(hipEventCreateWithFlags(&st.ev, hipEventDisableTiming));
    if (st.cap < P.bytes) {
      if (st.host) HIP_TRY(hipHostFree(st.host));
      st.host = nullptr;
      st.cap = 0;
      size_t want = align_up(P.bytes, (size_t)1 << 16);
      if (hipHostMalloc(&st.host, want, hipHostMallocDefault) != hipSuccess) {
        (void)hipGetLastError();
        st.host = nullptr;
        return fail(RW_ENOMEM, "hipHostMalloc(%zu) for a launch table failed", want);
      }
      st.cap = want;
    }
    fill_tables(P, items, st.host, ws);
    HIP_TRY(hipMemcpyAsync(ws, st.host, P.bytes, hipMemcpyHostToDevice, s));
    HIP_TRY(hipEventRecord(st.ev, s));
    st.pending = true;
  }
  return launch_group(P.launches, ws, P.map_off, P.qmap_off, s);
}

int rw_rocm_group_create(const rw_linear *items, size_t count, rw_group **out) {
  if (!out) return fail(RW_EINVAL, "out is NULL");
  *out = nullptr;
  if (count == 0 || !items) return fail(RW_EINVAL, "a group needs at least one item");
  int rc = check_group_items(items, count);
  if (rc) return rc;
  GroupPlan P = group_plan(items, count);
  if (P.order.empty()) return fail(RW_EINVAL, "every item has m = 0");
  const int device = items[0].w->device;
  HIP_TRY(hipSetDevice(device));
  rw_group *g = new rw_group;
  g->device = device;
  g->launches = P.launches;
  g->map_off = P.map_off;
  g->qmap_off = P.qmap_off;
  g->bytes = P.total;
  if (hipMalloc(&g->table, P.total) != hipSuccess) {
    (void)hipGetLastError();
    delete g;
    return fail(RW_ENOMEM, "hipMalloc(%zu) for a launch table failed", P.total);
  }
  std::vector<char> host(P.bytes);
  fill_tables(P, items, host.data(), g->table);
  hipError_t e = hipMemcpy(g->table, host.data(), P.bytes, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    (void)hipFree(g->table);
    delete g;
    return fail(RW_EHIP, "hipMemcpy: %s", hipGetErrorString(e));
  }
  *out = g;
  return RW_OK;
}

int rw_rocm_group_run(const rw_group *g, void *stream) {
  if (!g) return fail(RW_EINVAL, "group is NULL");
  HIP_TRY(hipSetDevice(g->device));
  return launch_group(g->launches, g->table, g->map_off, g->qmap_off, (hipStream_t)stream);
}

void rw_rocm_group_free(rw_group *g) {
  if (!g) return;
  if (hipSetDevice(g->device) == hipSuccess) (void)hipFree(g->table);
  (void)hipGetLastError();
  delete g;
}

int rw_rocm_dequant_rows(const rw_weight *w, size_t row0, size_t nrows, float *out) {
  if (!w) return fail(RW_EINVAL, "weight is NULL");
  if (row0 > w->n || nrows > w->n - row0)
    return fail(RW_EINVAL, "rows [%zu, %zu) out of range for %zu rows", row0, row0 + nrows, w->n);
  if (nrows == 0) return RW_OK;
  if (!out) return fail(RW_EINVAL, "out is NULL");
  HIP_TRY(hipSetDevice(w->device));
  CtxGuard g;
  int rc = ctx_acquire(w->device, &g.c);
  if (rc) return rc;
  size_t bytes = nrows * w->k * 4;
  rc = ctx_reserve(g.c, bytes);
  if (rc) return rc;
  size_t threads = nrows * (size_t)w->nb;
  dim3 grid((unsigned)cdiv(threads, 256));
#define RW_DEQ(DT) \
  hipLaunchKernelGGL(k_dequant<DT>, grid, dim3(256), 0, g.c->stream, w->view, (int)row0, (int)nrows, (float *)g.c->buf)
  switch (w->dtype) {
    case RW_Q4_0: RW_DEQ(RW_Q4_0); break;
    case RW_Q4_1: RW_DEQ(RW_Q4_1); break;
    case RW_Q5_0: RW_DEQ(RW_Q5_0); break;
    case RW_Q5_1: RW_DEQ(RW_Q5_1); break;
    default: RW_DEQ(RW_Q8_0); break;
  }
#undef RW_DEQ
  LAUNCH_TRY("k_dequant");
  HIP_TRY(hipMemcpyAsync(out, g.c->buf, bytes, hipMemcpyDeviceToHost, g.c->stream));
  HIP_TRY(hipStreamSynchronize(g.c->stream));
  return RW_OK;
}

int rw_rocm_quantize_acts(const float *a, size_t m, size_t k, int8_t *q, float *d, int32_t *sum) {
  if (k == 0 || k % QK) return fail(RW_EINVAL, "k must be a positive multiple of %d (got %zu)", QK, k);
  if (m == 0) return RW_OK;
  if (!a || !q || !d || !sum) return fail(RW_EINVAL, "NULL argument");
  int dev;
  int rc = current_device(&dev);
  if (rc) return rc;
  CtxGuard g;
  rc = ctx_acquire(dev, &g.c);
  if (rc) return rc;
  ActLayout L = act_layout_kind(m, k, false);
  size_t off_a = align_up(L.bytes, 256);
  rc = ctx_reserve(g.c, off_a + m * k * 4);
  if (rc) return rc;
  char *b = (char *)g.c->buf;
  HIP_TRY(hipMemcpyAsync(b + off_a, a, m * k * 4, hipMemcpyHostToDevice, g.c->stream));
  rc = launch_quantize((const float *)(b + off_a), m, k, L, b, g.c->stream);
  if (rc) return rc;
  std::vector<uint8_t> host(L.bytes);
  HIP_TRY(hipMemcpyAsync(host.data(), b, L.bytes, hipMemcpyDeviceToHost, g.c->stream));
  HIP_TRY(hipStreamSynchronize(g.c->stream));
  const int8_t *hq = (const int8_t *)(host.data() + L.off_qa);
  const float *hd = (const float *)(host.data() + L.off_da);
  const int32_t *hs = (const int32_t *)(host.data() + L.off_sa);
  for (size_t i = 0; i < m; ++i)
    for (int bl = 0; bl < L.nb; ++bl) {
      size_t slot = act_slot(L.nb, (int)(i / RG), bl, (int)(i % RG));
      for (int e = 0; e < QK; ++e) q[i * k + (size_t)bl * QK + e] = hq[slot * QK + mfma_pos(e)];
      d[i * L.nb + bl] = hd[slot];
      sum[i * L.nb + bl] = hs[slot];
    }
  return RW_OK;
}

int rw_rocm_block_dots(const rw_weight *w, const int8_t *qa, size_t m, int32_t *S) {
  if (!w) return fail(RW_EINVAL, "weight is NULL");
  if (m == 0) return RW_OK;
  if (!qa || !S) return fail(RW_EINVAL, "NULL argument");
  HIP_TRY(hipSetDevice(w->device));
  CtxGuard g;
  int rc = ctx_acquire(w->device, &g.c);
  if (rc) return rc;
  ActLayout L = act_layout_kind(m, w->k, false);
  size_t sbytes = m * w->n * (size_t)w->nb * 4;
  size_t off_s = align_up(L.bytes, 256);
  rc = ctx_reserve(g.c, off_s + sbytes);
  if (rc) return rc;
  std::vector<int8_t> host(L.bytes, 0);
  for (size_t i = 0; i < m; ++i)
    for (int bl = 0; bl < L.nb; ++bl) {
      size_t slot = act_slot(L.nb, (int)(i / RG), bl, (int)(i % RG));
      for (int e = 0; e < QK; ++e) host[slot * QK + mfma_pos(e)] = qa[i * w->k + (size_t)bl * QK + e];
    }
  char *b = (char *)g.c->buf;
  HIP_TRY(hipMemcpyAsync(b, host.data(), L.bytes, hipMemcpyHostToDevice, g.c->stream));
  ActView av = act_view(L, b);
  dim3 grid((unsigned)w->ngroups, (unsigned)L.mgroups, (unsigned)w->nb);
#define RW_BD(DT) \
  hipLaunchKernelGGL(k_block_dots<DT>, grid, dim3(64), 0, g.c->stream, w->view, av, (int)m, (int)w->n, (int32_t *)(b + off_s))
  switch (w->dtype) {
    case RW_Q4_0: RW_BD(RW_Q4_0); break;
    case RW_Q4_1: RW_BD(RW_Q4_1); break;
    case RW_Q5_0: RW_BD(RW_Q5_0); break;
    case RW_Q5_1: RW_BD(RW_Q5_1); break;
    default: RW_BD(RW_Q8_0); break;
  }
#undef RW_BD
  LAUNCH_TRY("k_block_dots");
  HIP_TRY(hipMemcpyAsync(S, b + off_s, sbytes, hipMemcpyDeviceToHost, g.c->stream));
  HIP_TRY(hipStreamSynchronize(g.c->stream));
  return RW_OK;
}

size_t rw_rocm_attention_workspace_size(size_t t_q, size_t t_kv, size_t n_state) {
  return attn_layout(t_q, t_kv, n_state).bytes;
}

int rw_rocm_attention_dev(const float *q, size_t ldq, const float *k, size_t ldk, const float *v, size_t ldv,
                          size_t t_q, size_t t_kv, size_t n_state, int n_head, int causal, float *out, size_t ldo,
                          void *workspace, size_t workspace_len, void *stream) {
  int rc = check_attn_args(q, ldq, k, ldk, v, ldv, t_q, t_kv, n_state, n_head, causal, out, ldo);
  if (rc) return rc;
  if (t_q == 0) return RW_OK;
  int dev;
  rc = current_device(&dev);
  if (rc) return rc;
  const AttnLayout L = attn_layout(t_q, t_kv, n_state);
  void *ws = workspace;
  WsHold hold;
  if (ws) {
    if (workspace_len < L.bytes) return fail(RW_EINVAL, "workspace of %zu bytes < %zu needed", workspace_len, L.bytes);
  } else {
    rc = stream_workspace(dev, stream, L.bytes, hold, &ws);
    if (rc) return rc;
  }
  return run_attention(q, ldq, k, ldk, v, ldv, t_q, t_kv, n_head, causal, out, ldo, L, ws, (hipStream_t)stream);
}

int rw_rocm_attention(const float *q, const float *k, const float *v, size_t t_q, size_t t_kv, size_t n_state,
                      int n_head, int causal, float *out) {
  int rc = check_attn_args(q, n_state, k, n_state, v, n_state, t_q, t_kv, n_state, n_head, causal, out, n_state);
  if (rc) return rc;
  if (t_q == 0) return RW_OK;
  int dev;
  rc = current_device(&dev);
  if (rc) return rc;
  CtxGuard g;
  rc = ctx_acquire(dev, &g.c);
  if (rc) return rc;
  Ctx *c = g.c;
  const AttnLayout L = attn_layout(t_q, t_kv, n_state);
  const size_t off_q = align_up(L.bytes, 256);
  const size_t off_k = align_up(off_q + t_q * n_state * 4, 256);
  const size_t off_v = align_up(off_k + t_kv * n_state * 4, 256);
  const size_t off_o = align_up(off_v + t_kv * n_state * 4, 256);
  rc = ctx_reserve(c, align_up(off_o + t_q * n_state * 4, 256));
  if (rc) return rc;
  char *b = (char *)c->buf;
  float *dq = (float *)(b + off_q), *dk = (float *)(b + off_k), *dv = (float *)(b + off_v), *dout = (float *)(b + off_o);
  HIP_TRY(hipMemcpyAsync(dq, q, t_q * n_state * 4, hipMemcpyHostToDevice, c->stream));
  if (t_kv) {
    HIP_TRY(hipMemcpyAsync(dk, k, t_kv * n_state * 4, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(hipMemcpyAsync(dv, v, t_kv * n_state * 4, hipMemcpyHostToDevice, c->stream));
  }
  rc = run_attention(dq, n_state, dk, n_state, dv, n_state, t_q, t_kv, n_head, causal, dout, n_state, L, b, c->stream);
  if (rc) {
    (void)hipStreamSynchronize(c->stream);
    return rc;
  }
  HIP_TRY(hipMemcpyAsync(out, dout, t_q * n_state * 4, hipMemcpyDeviceToHost, c->stream));
  HIP_TRY(hipStreamSynchronize(c->stream));
  return RW_OK;
}

int rw_rocm_decoder_create(const rw_decoder_params *params, size_t n_audio_ctx, rw_decoder **out) {
  if (!out) return fail(RW_EINVAL, "out is NULL");
  *out = nullptr;
  int rc = check_decoder_params(params);
  if (rc) return rc;
  if (n_audio_ctx == 0 || n_audio_ctx > (1u << 20)) return fail(RW_EINVAL, "n_audio_ctx = %zu", n_audio_ctx);
  HIP_TRY(hipSetDevice(params->token_embedding->device));
  rw_decoder *d = new rw_decoder();
  d->p = *params;
  d->layers.assign(params->layers, params->layers + params->n_layer);
  d->p.layers = d->layers.data();
  d->device = params->token_embedding->device;
  d->n = params->token_embedding->k;
  d->f = params->layers[0].fc1->n;
  d->n_audio = n_audio_ctx;
  const size_t kv = (size_t)params->n_layer * 2 * params->n_ctx * d->n * 4;
  if (hipMalloc(&d->self_kv, kv) != hipSuccess) {
    (void)hipGetLastError();
    d->self_kv = nullptr;
    delete d;
    return fail(RW_ENOMEM, "hipMalloc(%zu) for the self-attention caches failed", kv);
  }
  auto cross = std::make_shared<CrossKV>();
  cross->device = d->device;
  cross->n_audio = n_audio_ctx;
  cross->n = d->n;
  cross->n_layer = params->n_layer;
  cross->tkv_pad = (int)align_up(n_audio_ctx, ATT_KVB);
  cross->plane_bytes = align_up((size_t)params->n_head * ATT_DH * cross->tkv_pad * 2, 256);
  cross->layer_bytes = 4 * cross->plane_bytes;
  if (hipMalloc(&cross->buf, cross->layer_bytes * params->n_layer) != hipSuccess) {
    (void)hipGetLastError();
    cross->buf = nullptr;
    delete d;
    return fail(RW_ENOMEM, "hipMalloc for the cross-attention K/V failed");
  }
  d->cross = cross;
  *out = d;
  return RW_OK;
}

void rw_rocm_decoder_free(rw_decoder *d) { delete d; }

static int dec_reserve(rw_decoder *d, size_t bytes) {
  if (d->scratch_cap >= bytes) return RW_OK;
  if (d->scratch) HIP_TRY(hipFree(d->scratch));
  d->scratch = nullptr;
  d->scratch_cap = 0;
  const size_t want = align_up(bytes, (size_t)1 << 20);
  if (hipMalloc(&d->scratch, want) != hipSuccess) {
    (void)hipGetLastError();
    return fail(RW_ENOMEM, "hipMalloc(%zu) for decoder scratch failed", want);
  }
  d->scratch_cap = want;
  return RW_OK;
}

int rw_rocm_decoder_set_audio_dev(rw_decoder *d, const float *enc_out, void *stream) {
  if (!d || !enc_out) return fail(RW_EINVAL, "decoder or encoder output is NULL");
  if (!al16(enc_out)) return fail(RW_EINVAL, "the encoder output must be 16-byte aligned");
  if (d->cross.use_count() > 1) return fail(RW_EINVAL, "the cross K/V are shared with a fork; set audio on a fresh decoder");
  HIP_TRY(hipSetDevice(d->device));
  hipStream_t s = (hipStream_t)stream;
  const size_t T = d->n_audio, n = d->n;
  // k and v f32 for one layer, the activation workspace, then splitting
  const AttnLayout A = attn_layout(1, T, n);
  const size_t off_k = 0, off_v = align_up(T * n * 4, 256), off_act = align_up(off_v + T * n * 4, 256);
  const size_t bytes = align_up(off_act + act_layout(T, n).bytes, 256);
  int rc = dec_reserve(d, bytes);
  if (rc) return rc;
  char *b = (char *)d->scratch;
  float *kf = (float *)(b + off_k), *vf = (float *)(b + off_v);
  // every layer's K and V read the same encoder output: it is quantized
  // once (quantize_acts_i8 of the same rows gives the same values each
  // time), and a layer's K and V run as one two-weight launch where their
  // dtypes and k agree
  const ActLayout AL = act_layout(T, n);
  RW_TRY(launch_quantize(enc_out, T, n, AL, b + off_act, s));
  for (int l = 0; l < d->p.n_layer; ++l) {
    const rw_decoder_layer &L = d->layers[l];
    if (T > (size_t)GEMV_MAX_M && L.ck->dtype == L.cv->dtype && L.ck->k == L.cv->k) {
      const rw_weight *w2[2] = {L.ck, L.cv};
      const float *b2[2] = {nullptr, L.cv_b};  // the key has no bias
      float *o2[2] = {kf, vf};
      RW_TRY(run_gemm(w2, b2, o2, 2, act_view(AL, b + off_act), (int)T, s));
    } else {
      RW_TRY(run_product(L.ck, T, nullptr, kf, b + off_act, s));
      RW_TRY(run_product(L.cv, T, L.cv_b, vf, b + off_act, s));
    }
    const AttnPlanes cp = d->cross->planes(l);
    AttnPlanes P{nullptr, nullptr, cp.kh, cp.kl, cp.vh, cp.vl, A.tq_pad, cp.tkv_pad};
    const size_t nk = (size_t)d->p.n_head * cp.tkv_pad * 8;
    const int wk = (int)cdiv(nk, 256), wv = d->p.n_head * (int)cdiv(cp.tkv_pad, ATT_VT_KV);
    hipLaunchKernelGGL(k_attn_split, dim3((unsigned)(wk + wv)), dim3(256), 0, s, nullptr, (int)n, 0, kf, (int)n, vf,
                       (int)n, (int)T, P, d->p.n_head, 0, wk);
    LAUNCH_TRY("k_attn_split");
  }
  d->audio = true;
  d->n_past = 0;
  return RW_OK;
}

int rw_rocm_decoder_reset(rw_decoder *d) {
  if (!d) return fail(RW_EINVAL, "decoder is NULL");
  d->n_past = 0;
  return RW_OK;
}

int rw_rocm_decoder_n_past(const rw_decoder *d, size_t *n_past) {
  if (!d || !n_past) return fail(RW_EINVAL, "decoder or n_past is NULL");
  *n_past = d->n_past;
  return RW_OK;
}

int rw_rocm_decoder_fork(const rw_decoder *d, void *stream, rw_decoder **out) {
  if (!d || !out) return fail(RW_EINVAL, "decoder or out is NULL");
  *out = nullptr;
  HIP_TRY(hipSetDevice(d->device));
  rw_decoder *c = new rw_decoder();
  c->p = d->p;
  c->layers = d->layers;
  c->p.layers = c->layers.data();
  c->device = d->device;
  c->n = d->n, c->f = d->f, c->n_audio = d->n_audio, c->n_past = d->n_past;
  c->cross = d->cross;
  c->audio = d->audio;
  const size_t kv = (size_t)d->p.n_layer * 2 * d->p.n_ctx * d->n * 4;
  if (hipMalloc(&c->self_kv, kv) != hipSuccess) {
    (void)hipGetLastError();
    c->self_kv = nullptr;
    delete c;
    return fail(RW_ENOMEM, "hipMalloc(%zu) for the forked caches failed", kv);
  }
  if (d->n_past) {
    const size_t rows = d->n_past * d->n * 4;  // copy only the filled rows of each cache
    for (int l = 0; l < d->p.n_layer; ++l) {
      hipError_t e = hipMemcpyAsync(c->self_k(l), d->self_k(l), rows, hipMemcpyDeviceToDevice, (hipStream_t)stream);
      if (e == hipSuccess)
        e = hipMemcpyAsync(c->self_v(l), d->self_v(l), rows, hipMemcpyDeviceToDevice, (hipStream_t)stream);
      if (e != hipSuccess) {
        delete c;
        return fail(RW_EHIP, "fork copy: %s", hipGetErrorString(e));
      }
    }
  }
  *out = c;
  return RW_OK;
}

int rw_rocm_decoder_forward_hidden_dev(rw_decoder *d, const uint32_t *tokens, size_t n_tok, float *hidden,
                                       void *stream) {
  if (!d || !tokens || !hidden) return fail(RW_EINVAL, "decoder, tokens or hidden is NULL");
  if (n_tok == 0) return fail(RW_EINVAL, "n_tok must be positive");
  if (!d->audio) return fail(RW_EINVAL, "no audio window: call rw_rocm_decoder_set_audio_dev first");
  if (d->n_past + n_tok > (size_t)d->p.n_ctx)
    return fail(RW_EINVAL, "decoder context overflow: %zu + %zu > %d", d->n_past, n_tok, d->p.n_ctx);
  const size_t n_vocab = d->p.token_embedding->n;
  for (size_t i = 0; i < n_tok; ++i)
    if (tokens[i] >= n_vocab) return fail(RW_EINVAL, "token id %u out of range", tokens[i]);
  HIP_TRY(hipSetDevice(d->device));
  const DecScratch S = dec_scratch(d, n_tok);
  int rc = dec_reserve(d, S.bytes);
  if (rc) return rc;
  char *b = (char *)d->scratch;
  hipStream_t s = (hipStream_t)stream;
  HIP_TRY(hipMemcpyAsync(b + S.off_tok, tokens, n_tok * 4, hipMemcpyHostToDevice, s));
  rc = decoder_forward(&d, 1, false, n_tok, hidden, b, S, s);
  if (rc) return rc;
  d->n_past += n_tok;
  return RW_OK;
}

int rw_rocm_decoder_forward_beams_dev(rw_decoder *const *beams, size_t n_beams, const uint32_t *tokens,
                                      float *hidden, void *stream) {
  if (!beams || !tokens || !hidden) return fail(RW_EINVAL, "beams, tokens or hidden is NULL");
  if (n_beams < 1 || n_beams > (size_t)ATT_MAX_BEAMS)
    return fail(RW_EINVAL, "n_beams = %zu: between 1 and %d beams per step", n_beams, ATT_MAX_BEAMS);
  rw_decoder *d = beams[0];
  for (size_t i = 0; i < n_beams; ++i) {
    const rw_decoder *e = beams[i];
    if (!e) return fail(RW_EINVAL, "beam %zu is NULL", i);
    if (!e->audio) return fail(RW_EINVAL, "beam %zu: no audio window: call rw_rocm_decoder_set_audio_dev first", i);
    if (e->cross != d->cross || e->p.token_embedding != d->p.token_embedding)
      return fail(RW_EINVAL, "beam %zu is not a fork of beam 0's decoder (another model or audio window)", i);
    if (e->n_past != d->n_past)
      return fail(RW_EINVAL, "beam %zu has %zu cached tokens, beam 0 has %zu", i, e->n_past, d->n_past);
    for (size_t j = 0; j < i; ++j)
      if (beams[j] == e) return fail(RW_EINVAL, "beam %zu is listed twice", i);
  }
  if (d->n_past + 1 > (size_t)d->p.n_ctx)
    return fail(RW_EINVAL, "decoder context overflow: %zu + 1 > %d", d->n_past, d->p.n_ctx);
  const size_t n_vocab = d->p.token_embedding->n;
  for (size_t i = 0; i < n_beams; ++i)
    if (tokens[i] >= n_vocab) return fail(RW_EINVAL, "token id %u out of range", tokens[i]);
  HIP_TRY(hipSetDevice(d->device));
  const DecScratch S = dec_scratch(d, n_beams, true);
  int rc = dec_reserve(d, S.bytes);
  if (rc) return rc;
  char *b = (char *)d->scratch;
  hipStream_t s = (hipStream_t)stream;
  HIP_TRY(hipMemcpyAsync(b + S.off_tok, tokens, n_beams * 4, hipMemcpyHostToDevice, s));
  rc = decoder_forward(beams, n_beams, true, n_beams, hidden, b, S, s);
  if (rc) return rc;
  for (size_t i = 0; i < n_beams; ++i) beams[i]->n_past += 1;
  return RW_OK;
}

struct TopkLayout {
  int nc;
  size_t off_pm, off_ps, off_cv, off_ci, bytes;
};
static TopkLayout topk_layout(size_t rows, size_t n_vocab, size_t k) {
  TopkLayout L{};
  L.nc = (int)cdiv(n_vocab, TOPK_CHUNK);
  const size_t np = rows * L.nc, nk = np * (2 * k - 1);  // 2k - 1 picks per chunk
  L.off_pm = 0;
  L.off_ps = align_up(np * 4, 256);
  L.off_cv = align_up(L.off_ps + np * 4, 256);
  L.off_ci = align_up(L.off_cv + nk * 4, 256);
  L.bytes = align_up(L.off_ci + nk * 4, 256);
  return L;
}

size_t rw_rocm_logits_topk_workspace_size(size_t rows, size_t n_vocab, size_t k) {
  if (rows == 0 || n_vocab == 0 || k == 0) return 0;
  return topk_layout(rows, n_vocab, k).bytes;
}

int rw_rocm_logits_topk_dev(const float *logits, size_t rows, size_t n_vocab, size_t k, uint32_t *ids,
                            float *logprobs, void *workspace, size_t workspace_len, void *stream) {
  if (rows == 0) return RW_OK;
  if (!logits || !ids || !logprobs) return fail(RW_EINVAL, "logits, ids or logprobs is NULL");
  if (k < 1 || k > (size_t)TOPK_MAX) return fail(RW_EINVAL, "k = %zu: between 1 and %d", k, TOPK_MAX);
  if (n_vocab == 0 || n_vocab > (size_t)TOPK_CHUNK * TOPK_MAX_CHUNKS)
    return fail(RW_EINVAL, "n_vocab = %zu: between 1 and %d", n_vocab, TOPK_CHUNK * TOPK_MAX_CHUNKS);
  if (rows > 65535) return fail(RW_EINVAL, "rows = %zu: at most 65535", rows);
  int dev;
  int rc = current_device(&dev);
  if (rc) return rc;
  const TopkLayout L = topk_layout(rows, n_vocab, k);
  void *ws = workspace;
  WsHold hold;
  if (ws) {
    if (workspace_len < L.bytes) return fail(RW_EINVAL, "workspace of %zu bytes < %zu needed", workspace_len, L.bytes);
  } else {
    rc = stream_workspace(dev, stream, L.bytes, hold, &ws);
    if (rc) return rc;
  }
  char *b = (char *)ws;
  float *pm = (float *)(b + L.off_pm), *ps = (float *)(b + L.off_ps), *cv = (float *)(b + L.off_cv);
  int *ci = (int *)(b + L.off_ci);
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)L.nc, (unsigned)rows);
  hipLaunchKernelGGL(k_topk_stats, grid, dim3(256), 0, s, logits, (int)n_vocab, pm, ps);
  LAUNCH_TRY("k_topk_stats");
  hipLaunchKernelGGL(k_topk_chunk, grid, dim3(256), 0, s, logits, (int)n_vocab, (int)k, pm, ps, cv, ci);
  LAUNCH_TRY("k_topk_chunk");
  hipLaunchKernelGGL(k_topk_merge, dim3((unsigned)rows), dim3(256), 0, s, L.nc, (int)k, (int)n_vocab, pm, ps, cv,
                     ci, ids, logprobs);
  LAUNCH_TRY("k_topk_merge");
  return RW_OK;
}

size_t rw_rocm_encoder_layer_workspace_size(const rw_encoder_layer *layer, size_t t) {
  if (!layer || !layer->q || !layer->fc1) return 0;
  return layer_layout(layer->q->k, layer->fc1->n, t).bytes;
}

int rw_rocm_encoder_layer_dev(const rw_encoder_layer *layer, float *x, size_t t, void *workspace,
                              size_t workspace_len, void *stream) {
  int rc = check_layer(layer, t);
  if (rc) return rc;
  if (!x || !al16(x)) return fail(RW_EINVAL, "x must be a 16-byte aligned device pointer");
  HIP_TRY(hipSetDevice(layer->q->device));
  const size_t need = layer_layout(layer->q->k, layer->fc1->n, t).bytes;
  void *ws = workspace;
  WsHold hold;
  if (ws) {
    if (workspace_len < need) return fail(RW_EINVAL, "workspace of %zu bytes < %zu needed", workspace_len, need);
  } else {
    rc = stream_workspace(layer->q->device, stream, need, hold, &ws);
    if (rc) return rc;
  }
  return run_encoder_layer(layer, x, t, ws, (hipStream_t)stream);
}

}  // extern "C"
