// Quantisation kernels for the TCFP-12 path on gfx950.
//
// Built with -ffp-contract=off: the reference evaluates every product and
// sum as a separately rounded torch op (tcfp/nn/__init__.py:364, 378-383,
// tcfp/kernels.py:1870-1873), and the codes / error buffers here must match
// it bit for bit, so no multiply-add may be fused.
//
// HBM layout: inputs are read once per pass with 16-byte vector loads; each
// thread owns whole 8-element vectors, so the in-place error-feedback update
// of a vector is done by the thread that read it.
#include <algorithm>
#include <cstring>
#include <mutex>

#include "common.h"

using namespace tcfp;

namespace {

// Per-tensor reductions.  Each workgroup of a reducing kernel stores its
// partial max |x| (as float bits: monotone for non-negative floats, and any
// NaN sorts above +inf, so torch.max's NaN propagation is kept) into its own
// slot of a workspace array with a plain store.  The kernel that consumes the
// scale re-reduces every slot in every workgroup (at most 8 KiB, served from
// L2), so the two launches need nothing but stream order: no atomics, no
// fences, no zero-at-rest requirement, and the result is deterministic.
constexpr int kMaxParts = 2048;
struct PartWs {
  uint32_t a[kMaxParts];  // partial amax of the first reduction
  uint32_t b[kMaxParts];  // partial amax of the residual (dual quantisation)
  // NF-aware scaling: per-workgroup shifted sums of the first pass,
  // sum(v - v0) and sum((v - v0)^2) in fp64 (v0 = the tensor's first element)
  double s1[kMaxParts];
  double s2[kMaxParts];
  // W_hi target (before any EMA) published by workgroup 0 of the W_hi pass
  // for the residual pass, which then skips re-reducing the partials
  float hi_tgt;
  // GELU amax rule: applies (0/1) and the amax bits it gives
  uint32_t gelu_rule[2];
  uint32_t pad2[61];
};

constexpr int kThreads = 256;

int g_num_cu = 0;

int num_cu() {
  if (g_num_cu == 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
        n > 0)
      g_num_cu = n;
    else
      g_num_cu = 256;
  }
  return g_num_cu;
}

inline int grid_for(int64_t work_items, int per_cu) {
  int64_t g = (work_items + kThreads - 1) / kThreads;
  int64_t cap = int64_t(num_cu()) * per_cu;
  if (g > cap) g = cap;
  if (g < 1) g = 1;
  return int(g);
}

// Workgroups of a kernel that writes partials: about four 8-element vectors
// per thread, never more than the workspace holds.
inline int parts_for(int64_t nvec) {
  int64_t g = (nvec + 4 * kThreads - 1) / (4 * kThreads);
  const int64_t cap = std::min<int64_t>(kMaxParts, int64_t(num_cu()) * 4);
  if (g > cap) g = cap;
  if (g < 1) g = 1;
  return int(g);
}

inline int launch_status() { return hipGetLastError() == hipSuccess ? TCFP_OK : TCFP_ERR_HIP; }

// ---- vector loads: 8 consecutive elements as float -----------------------
TCFP_DEV void load8(const float* p, float v[8]) {
  float4 a = *reinterpret_cast<const float4*>(p);
  float4 b = *reinterpret_cast<const float4*>(p + 4);
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}
TCFP_DEV void load8(const uint16_t* p, float v[8]) {
  uint4 a = *reinterpret_cast<const uint4*>(p);
  uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = __uint_as_float(w[i] << 16);
    v[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
  }
}
TCFP_DEV float load1(const float* p) { return *p; }
TCFP_DEV float load1(const uint16_t* p) { return bf16_to_f32(*p); }

TCFP_DEV void store8(float* p, const float v[8]) {
  *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
  *reinterpret_cast<float4*>(p + 4) = make_float4(v[4], v[5], v[6], v[7]);
}


template <int FMT>
TCFP_DEV uint2 encode8(const float v[8]) {
#ifdef TCFP_SW_CVT
  return make_uint2(sw4_fp8<FMT>(v[0], v[1], v[2], v[3]), sw4_fp8<FMT>(v[4], v[5], v[6], v[7]));
#else
  return make_uint2(cvt4_fp8<FMT>(v[0], v[1], v[2], v[3]), cvt4_fp8<FMT>(v[4], v[5], v[6], v[7]));
#endif
}

template <int FMT>
TCFP_DEV uint32_t encode4(float a, float b, float c, float d) {
#ifdef TCFP_SW_CVT
  return sw4_fp8<FMT>(a, b, c, d);
#else
  return cvt4_fp8<FMT>(a, b, c, d);
#endif
}

template <int FMT>
TCFP_DEV uint32_t encode1(float v) {
#ifdef TCFP_SW_CVT
  return f32_to_fp8<FMT>(v);
#else
  return cvt4_fp8<FMT>(v, 0.f, 0.f, 0.f) & 0xFFu;
#endif
}

TCFP_DEV uint32_t byte_of(uint2 c, int j) { return ((j < 4 ? c.x : c.y) >> (8 * (j & 3))) & 0xFFu; }

// ---- per-tensor scale rule (tcfp/core.py:100-101, 105) ---------------------
// amax is NaN-propagating; clamp(min=1e-12) keeps NaN; the reciprocal and the
// product with FP8_MAX are each rounded to the input dtype.
TCFP_DEV void scale_from_amax(float amax, bool bf16_rule, float fmax, float* scale, float* inv) {
  float a = amax;
  if (bf16_rule) {
    const float lo = round_bf16(1e-12f);
    a = (a != a) ? a : fmaxf(a, lo);
    float rcp = round_bf16(__fdiv_rn(1.0f, a));
    *scale = round_bf16(__fmul_rn(rcp, fmax));
  } else {
    a = (a != a) ? a : fmaxf(a, 1e-12f);
    float rcp = __fdiv_rn(1.0f, a);
    *scale = __fmul_rn(rcp, fmax);
  }
  *inv = __fdiv_rn(1.0f, *scale);
}

// Workgroup-wide uint max (256 threads), returned to every thread.  `red`
// is the caller's LDS scratch: one call per array between barriers.
TCFP_DEV uint32_t block_umax_all(uint32_t m, uint32_t* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = umax(m, uint32_t(__shfl_xor(int(m), o, 64)));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  m = red[0];
#pragma unroll
  for (int i = 1; i < kThreads / 64; ++i) m = umax(m, red[i]);
  return m;
}

// Workgroup-wide uint max over NT threads (a multiple of 64), returned to
// every thread; `red` holds NT / 64 words.
template <int NT>
TCFP_DEV uint32_t block_umax_nt(uint32_t m, uint32_t* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = umax(m, uint32_t(__shfl_xor(int(m), o, 64)));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  m = red[0];
#pragma unroll
  for (int i = 1; i < NT / 64; ++i) m = umax(m, red[i]);
  return m;
}

// max over the partials p[0 .. g) written by the previous launch.
TCFP_DEV float reduce_parts(const uint32_t* __restrict__ p, int g, uint32_t* red) {
  uint32_t m = 0;
  for (int i = threadIdx.x; i < g; i += kThreads) m = umax(m, p[i]);
  return __uint_as_float(block_umax_all(m, red));
}

// The scale a per-tensor consumer kernel works with: the explicit one, or
// the amax rule over the partials.  Workgroup 0 publishes (scale, inv);
// `bid` is the workgroup's index when a launch serves several tensors
// (-1: blockIdx.x).
TCFP_DEV float consumer_scale(const float* scale_in, const uint32_t* part, int g, bool bf16_rule,
                              float fmax, float* scale_out, float* inv_out, uint32_t* red,
                              int bid = -1) {
  float s, inv;
  if (scale_in) {
    s = *scale_in;
    inv = __fdiv_rn(1.0f, s);
  } else {
    scale_from_amax(reduce_parts(part, g, red), bf16_rule, fmax, &s, &inv);
  }
  if ((bid < 0 ? int(blockIdx.x) : bid) == 0 && threadIdx.x == 0) {
    if (scale_out) *scale_out = s;
    if (inv_out) *inv_out = inv;
  }
  return s;
}

// Delayed ("predictive dual-track") per-tensor scaling of one weight
// (tcfp/core.py:341-403, tcfp/nn/__init__.py:250-309).  `on == 0` selects
// the plain per-tensor rule.  The previous EMA values are read from
// amax_prev / ratio_prev (null: not tracked yet) and the new ones are
// written to amax_out / ratio_out by workgroup 0 of the last pass, so the
// state a launch reads is never the state it writes.
struct Delayed {
  const float* amax_prev;
  const float* ratio_prev;
  float* amax_out;
  float* ratio_out;
  float a, b;    // fp32(ema_decay), fp32(1 - ema_decay)
  int on;
  int validate;  // measure the residual amax this step (else predict it)
};

// torch's `d * prev + (1 - d) * cur` on fp32 tensors: three rounded ops.
TCFP_DEV float ema_f32(float prev, float cur, float a, float b) {
  return __fadd_rn(__fmul_rn(a, prev), __fmul_rn(b, cur));
}
TCFP_DEV float clamp_min_nan(float v, float lo) { return (v != v) ? v : fmaxf(v, lo); }
// (FP8_MAX / v).to(float32) for an fp32 tensor v: reciprocal, then product;
// inv = 1 / scale (to_fp8_e4m3 with an explicit scale, tcfp/core.py:99-106).
TCFP_DEV void scale_of(float v, float fmax, float* s, float* inv) {
  *s = __fmul_rn(__fdiv_rn(1.0f, v), fmax);
  *inv = __fdiv_rn(1.0f, *s);
}
// get_delayed_amax (tcfp/core.py:341-356) of this step's clamped amax.
TCFP_DEV float delayed_amax(const Delayed& d, float cur) {
  return d.amax_prev ? ema_f32(*d.amax_prev, cur, d.a, d.b) : cur;
}

// The W_hi scale rule.  `s1 == nullptr`: the amax rule (tcfp/core.py:100-101).
// Otherwise NF-aware scaling (to_fp8_e4m3_nf_aware, tcfp/core.py:161-193):
// the target is sigma * std(v) with the unbiased std (torch.std's default
// correction), or the amax when that std is below 1e-6; under delayed
// scaling the target feeds the EMA in place of the amax (tcfp/nn/__init__.py:
// 263-275).  `sr`: W_hi codes are rounded stochastically (stochastic=True).
struct HiRule {
  const double* s1;  // per-workgroup sum(v - v0) of the first pass
  const double* s2;  // per-workgroup sum((v - v0)^2)
  int64_t n;         // element count
  float sigma;       // fp32(sigma_factor): `sigma_factor * std` on an fp32 tensor
  int sr;
};

// Workgroup-wide fp64 sum (256 threads) in a fixed order, returned to every
// thread; `red` holds kThreads / 64 doubles.
TCFP_DEV double block_dsum_all(double v, double* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  double s = red[0];
#pragma unroll
  for (int i = 1; i < kThreads / 64; ++i) s += red[i];
  return s;
}

// The unbiased standard deviation from the shifted sums: fp64 arithmetic,
// then one rounding to fp32.  Fewer than two elements give NaN, as torch.std
// does; a non-finite element gives NaN through the sums.
TCFP_DEV float std_from_sums(double a1, double a2, int64_t n) {
  if (n < 2) return __builtin_nanf("");
  const double nd = double(n);
  double var = (a2 - a1 * (a1 / nd)) / (nd - 1.0);
  if (var < 0.0) var = 0.0;  // rounding of a near-constant tensor
  return float(sqrt(var));
}

// This step's W_hi target (before any EMA): the clamped amax, or the
// NF-aware sigma target.  Every workgroup re-reduces the partials in the same
// order, so all of them agree bit for bit.  `rd` holds 2 * kThreads / 64
// doubles.
TCFP_DEV float hi_target(const HiRule& hr, const uint32_t* __restrict__ pa, int ga,
                         uint32_t* red, double* rd) {
  if (!hr.s1) return clamp_min_nan(reduce_parts(pa, ga, red), 1e-12f);
  // all three partial arrays are loaded before any is reduced, so their
  // latencies overlap
  uint32_t m = 0;
  double a1 = 0.0, a2 = 0.0;
  for (int i = threadIdx.x; i < ga; i += kThreads) {
    m = umax(m, pa[i]);
    a1 += hr.s1[i];
    a2 += hr.s2[i];
  }
  const float amax = clamp_min_nan(__uint_as_float(block_umax_all(m, red)), 1e-12f);
  a1 = block_dsum_all(a1, rd);
  a2 = block_dsum_all(a2, rd + kThreads / 64);
  const float sd = clamp_min_nan(std_from_sums(a1, a2, hr.n), 1e-12f);
  return sd < 1e-6f ? amax : __fmul_rn(hr.sigma, sd);
}

// Eight elements of x (+ ef) starting at element 8*i.
template <typename InT, bool HAS_EF>
TCFP_DEV void load_w8(const InT* __restrict__ x, const float* __restrict__ ef, int64_t i,
                      float W[8], float v[8]) {
  load8(x + i * 8, W);
  if constexpr (HAS_EF) {
    float e[8];
    load8(ef + i * 8, e);
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = W[j] + e[j];
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = W[j];
  }
}

// ===========================================================================
// Per-tensor quantisation
// ===========================================================================

// Partial max |x (+ ef)| of this workgroup's share -> part[blockIdx.x].
// Four vectors are loaded before any is reduced, so each thread keeps 64 or
// 128 bytes in flight.  STATS (NF-aware scaling) also writes the partial
// sums of (v - v0) and (v - v0)^2 in fp64 to s1p / s2p, v0 being the first
// element: the shift keeps the variance free of cancellation when the mean
// is large against the spread.
// (body: workgroup `bid` of `nbk`; a batched launch runs it for one of
// several tensors)
template <typename InT, bool HAS_EF, bool STATS>
TCFP_DEV void amax_part_body(const InT* __restrict__ x,
                                                             const float* __restrict__ ef,
                                                             int64_t n, uint32_t* __restrict__ part,
                                                             double* __restrict__ s1p,
                                                             double* __restrict__ s2p,
                                                             const int bid, const int nbk,
                                                             uint32_t* red, double* rd) {
  uint32_t m = 0;
  double a1 = 0.0, a2 = 0.0, v0 = 0.0;
  if constexpr (STATS) {
    if (n > 0) {
      float f = load1(x);
      if constexpr (HAS_EF) f = f + ef[0];
      v0 = double(f);
    }
  }
  auto acc = [&](float v) {
    m = umax(m, absbits(v));
    if constexpr (STATS) {
      const double d = double(v) - v0;
      a1 += d;
      a2 = fma(d, d, a2);
    }
  };
  const int64_t nvec = n >> 3;
  const int64_t stride = int64_t(nbk) * kThreads;
  int64_t i = int64_t(bid) * kThreads + threadIdx.x;
  for (; i + 3 * stride < nvec; i += 4 * stride) {
    float W[4][8], v[4][8];
#pragma unroll
    for (int u = 0; u < 4; ++u) load_w8<InT, HAS_EF>(x, ef, i + u * stride, W[u], v[u]);
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc(v[u][j]);
  }
  for (; i < nvec; i += stride) {
    float W[8], v[8];
    load_w8<InT, HAS_EF>(x, ef, i, W, v);
#pragma unroll
    for (int j = 0; j < 8; ++j) acc(v[j]);
  }
  for (int64_t t = nvec * 8 + int64_t(bid) * kThreads + threadIdx.x; t < n; t += stride) {
    float v = load1(x + t);
    if constexpr (HAS_EF) v = v + ef[t];
    acc(v);
  }
  m = block_umax_all(m, red);
  if constexpr (STATS) {
    a1 = block_dsum_all(a1, rd);
    a2 = block_dsum_all(a2, rd + kThreads / 64);
  }
  if (threadIdx.x == 0) {
    part[bid] = m;
    if constexpr (STATS) {
      s1p[bid] = a1;
      s2p[bid] = a2;
    }
  }
}

template <typename InT, bool HAS_EF, bool STATS>
__global__ __launch_bounds__(kThreads) void amax_part_kernel(const InT* __restrict__ x,
                                                             const float* __restrict__ ef,
                                                             int64_t n, uint32_t* __restrict__ part,
                                                             double* __restrict__ s1p,
                                                             double* __restrict__ s2p) {
  __shared__ uint32_t red[kThreads / 64];
  __shared__ double rd[2 * (kThreads / 64)];
  amax_part_body<InT, HAS_EF, STATS>(x, ef, n, part, s1p, s2p, int(blockIdx.x), int(gridDim.x),
                                     red, rd);
}

// Pass 1 of the dual quantisation under the amax rule on large tensors: the
// partial max |v| of v = x (+ ef) as amax_part_kernel, and also the
// "candidates" for the residual amax: every v with |v| >= amax * 4/7 (and
// some smaller ones) is stored into this workgroup's region of `vals` (cap
// floats), their number into cnt[blockIdx.x] (more than cap: overflow).
// The workgroup takes its vectors in rounds of kCandCh per thread; after
// each round its running maximum M is reduced and the round's values with
// |v| >= 0.5714 M are stored (M <= amax and 0.5714 < 4/7, so nothing with
// |v| >= amax * 4/7 is missed), placed by a wave scan of the per-lane
// counts and one LDS atomic per wave.
struct CandOut {
  float* vals;    // region of workgroup b: vals + b * cap
  uint32_t* cnt;  // per-workgroup count
  int cap;
};
constexpr int kCandCh = 4;
template <typename InT, bool HAS_EF>
__global__ __launch_bounds__(kThreads) void amax_cand_kernel(const InT* __restrict__ x,
                                                             const float* __restrict__ ef,
                                                             int64_t n, uint32_t* __restrict__ part,
                                                             CandOut co) {
  __shared__ uint32_t red[kThreads / 64];
  __shared__ uint32_t ncand;
  if (threadIdx.x == 0) ncand = 0;
  float* const region = co.vals + int64_t(blockIdx.x) * co.cap;
  const int lane = threadIdx.x & 63;
  uint32_t mw = 0;  // the workgroup's running maximum (uniform)
  // store v[j] (j < nv) with |v| >= 0.5714 * the running maximum.  Zeros
  // are never stored: their residual is zero, below any decisive maximum,
  // and while the running maximum is still 0 they would all pass (a zero
  // head of a tensor would fill the region and force the full pass).
  auto emit = [&](const float* v, int nv) {
    const float thr = __uint_as_float(mw) * 0.5714f;
    uint64_t mask = 0;
    for (int j = 0; j < nv; ++j) mask |= uint64_t(fabsf(v[j]) >= thr && v[j] != 0.0f) << j;
    const int c = __builtin_popcountll(mask);
    int incl = c;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int t = __shfl_up(incl, d, 64);
      if (lane >= d) incl += t;
    }
    const int tot = __shfl(incl, 63, 64);
    uint32_t base = 0;
    if (lane == 0 && tot > 0) base = atomicAdd(&ncand, uint32_t(tot));
    base = uint32_t(__shfl(int(base), 0, 64));
    uint32_t pos = base + uint32_t(incl - c);
    while (mask) {
      const int j = __builtin_ctzll(mask);
      mask &= mask - 1;
      if (pos < uint32_t(co.cap)) region[pos] = v[j];
      ++pos;
    }
  };
  const int64_t nvec = n >> 3;
  const int64_t stride = int64_t(gridDim.x) * kThreads;
  const int64_t i0 = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  const int64_t w0 = int64_t(blockIdx.x) * kThreads;  // the workgroup's first vector
  // (workgroup-uniform trip count: block_umax_all synchronises)
  for (int64_t r = 0; w0 + r * kCandCh * stride < nvec; ++r) {
    float W[kCandCh][8], v[kCandCh][8];
    int nv = 0;
    uint32_t mt = 0;
#pragma unroll
    for (int u = 0; u < kCandCh; ++u) {
      const int64_t iv = i0 + (r * kCandCh + u) * stride;
      if (iv < nvec) {
        load_w8<InT, HAS_EF>(x, ef, iv, W[u], v[u]);
        nv = 8 * (u + 1);
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) v[u][j] = 0.0f;
      }
    }
#pragma unroll
    for (int u = 0; u < kCandCh; ++u)
#pragma unroll
      for (int j = 0; j < 8; ++j) mt = umax(mt, absbits(v[u][j]));
    mw = umax(mw, block_umax_all(mt, red));
    emit(&v[0][0], nv);
    __syncthreads();  // red is reused by the next round's reduction
  }
  // the last n % 8 elements (workgroup 0)
  if (blockIdx.x == 0) {
    const int64_t t = nvec * 8 + threadIdx.x;
    float v = 0.0f;
    uint32_t mt = 0;
    const bool live = t < n;
    if (live) {
      v = load1(x + t);
      if constexpr (HAS_EF) v = v + ef[t];
      mt = absbits(v);
    }
    mw = umax(mw, block_umax_all(mt, red));
    emit(&v, live ? 1 : 0);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    part[blockIdx.x] = mw;
    co.cnt[blockIdx.x] = ncand;
  }
}

// ---- GELU producers ---------------------------------------------------------
// gelu_f32 / gelu_bwd_f32 (common.h) evaluate torch's GELU bit for bit.

// act = gelu(h) (written out unless act is null) and this workgroup's
// partial max |act| -> part[blockIdx.x], the producer of a per-tensor
// quantisation of act (which may recompute act from h instead of reading it).
// 512-thread workgroups: the partial count is capped, and the erf makes the
// pass VALU-heavy, so each CU needs eight waves per SIMD to overlap the
// arithmetic with the memory traffic.
constexpr int kGeluThreads = 512;
// workgroups of the GELU passes over n elements: up to kMaxParts, two
// 8-element vectors per thread at least (measured: 2048 x 512 threads 42
// us, 1024 x 512 threads 44.5 us for 32 Mi elements)
int gelu_grid(int64_t n) {
  return int(std::max<int64_t>(
      1, std::min<int64_t>(kMaxParts, ((n + 7) / 8 + 2 * kGeluThreads - 1) / (2 * kGeluThreads))));
}
__global__ __launch_bounds__(kGeluThreads) void gelu_amax_kernel(const float* __restrict__ h,
                                                                 int64_t n, float* __restrict__ act,
                                                                 uint32_t* __restrict__ part) {
  __shared__ uint32_t red[kGeluThreads / 64];
  uint32_t m = 0;
  const int64_t nvec = n >> 3;
  const int64_t stride = int64_t(gridDim.x) * kGeluThreads;
  auto body = [&](const float v[8], int64_t i) {
    float g[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) g[j] = gelu_f32(v[j]);
    if (act) store8(act + i * 8, g);
    // the max after the stores, over all eight (measured faster than
    // folding each value in as it is produced)
    const uint32_t m01 = umax(absbits(g[0]), absbits(g[1])), m23 = umax(absbits(g[2]), absbits(g[3]));
    const uint32_t m45 = umax(absbits(g[4]), absbits(g[5])), m67 = umax(absbits(g[6]), absbits(g[7]));
    m = umax(m, umax(umax(m01, m23), umax(m45, m67)));
  };
  // one vector per step: the erf branches per element, and deeper unrolling
  // measured slower (52 vs 41 us for 32 Mi elements with four in flight)
  for (int64_t i = int64_t(blockIdx.x) * kGeluThreads + threadIdx.x; i < nvec; i += stride) {
    float v[8];
    load8(h + i * 8, v);
    body(v, i);
  }
  for (int64_t t = nvec * 8 + int64_t(blockIdx.x) * kGeluThreads + threadIdx.x; t < n;
       t += stride) {
    const float g = gelu_f32(h[t]);
    if (act) act[t] = g;
    m = umax(m, absbits(g));
  }
  m = block_umax_nt<kGeluThreads>(m, red);
  if (threadIdx.x == 0) part[blockIdx.x] = m;
}

// grad = gelu_bwd(h, dy) (written out) and this workgroup's partial max
// |grad| -> part[blockIdx.x]: the producer of the per-tensor quantisation of
// a GELU's input gradient.
// dy and grad may be the same buffer (each element is read, then written,
// by the same lane).
__global__ __launch_bounds__(kGeluThreads) void gelu_bwd_amax_kernel(
    const float* dy, const float* __restrict__ h, int64_t n, float* grad,
    uint32_t* __restrict__ part) {
  __shared__ uint32_t red[kGeluThreads / 64];
  uint32_t m = 0;
  const int64_t nvec = n >> 3;
  const int64_t stride = int64_t(gridDim.x) * kGeluThreads;
  for (int64_t i = int64_t(blockIdx.x) * kGeluThreads + threadIdx.x; i < nvec; i += stride) {
    float v[8], hv[8];
    load8(dy + i * 8, v);
    load8(h + i * 8, hv);
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = gelu_bwd_f32(hv[j], v[j]);
    store8(grad + i * 8, v);
    const uint32_t m01 = umax(absbits(v[0]), absbits(v[1])), m23 = umax(absbits(v[2]), absbits(v[3]));
    const uint32_t m45 = umax(absbits(v[4]), absbits(v[5])), m67 = umax(absbits(v[6]), absbits(v[7]));
    m = umax(m, umax(umax(m01, m23), umax(m45, m67)));
  }
  for (int64_t t = nvec * 8 + int64_t(blockIdx.x) * kGeluThreads + threadIdx.x; t < n;
       t += stride) {
    const float v = gelu_bwd_f32(h[t], dy[t]);
    grad[t] = v;
    m = umax(m, absbits(v));
  }
  m = block_umax_nt<kGeluThreads>(m, red);
  if (threadIdx.x == 0) part[blockIdx.x] = m;
}

// out = a * b and this workgroup's partial max |out| -> part[blockIdx.x]
// (the GELU backward from its saved derivative factor).  out may be a.
__global__ __launch_bounds__(kGeluThreads) void mul_amax_kernel(const float* a,
                                                                const float* __restrict__ b,
                                                                int64_t n, float* out,
                                                                uint32_t* __restrict__ part) {
  __shared__ uint32_t red[kGeluThreads / 64];
  uint32_t m = 0;
  const int64_t nvec = n >> 3;
  const int64_t stride = int64_t(gridDim.x) * kGeluThreads;
  for (int64_t i = int64_t(blockIdx.x) * kGeluThreads + threadIdx.x; i < nvec; i += stride) {
    float v[8], w[8];
    load8(a + i * 8, v);
    load8(b + i * 8, w);
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = v[j] * w[j];
    store8(out + i * 8, v);
#pragma unroll
    for (int j = 0; j < 8; ++j) m = umax(m, absbits(v[j]));
  }
  for (int64_t t = nvec * 8 + int64_t(blockIdx.x) * kGeluThreads + threadIdx.x; t < n;
       t += stride) {
    const float v = a[t] * b[t];
    out[t] = v;
    m = umax(m, absbits(v));
  }
  m = block_umax_nt<kGeluThreads>(m, red);
  if (threadIdx.x == 0) part[blockIdx.x] = m;
}

// ---- premises of the GELU amax rule ---------------------------------------
// Checked once per device over every fp32 input: (1) gelu_f32 is
// non-decreasing on [+0, +inf] (each positive bit pattern against the next);
// (2) T = max |gelu_f32(x)| over the negative numbers from -0 to the most
// negative finite value.  The check kernel writes per-workgroup results, a
// one-workgroup finaliser reduces them and publishes `done` last.
constexpr int kPremiseWgs = 1024;
struct GeluPremise {
  uint32_t done;
  uint32_t violations;
  uint32_t t_bits;
  uint32_t pad;
  uint32_t wg_viol[kPremiseWgs];
  uint32_t wg_t[kPremiseWgs];
};
__device__ GeluPremise g_gelu_premise;

__global__ __launch_bounds__(kThreads) void gelu_premise_check_kernel() {
  __shared__ uint32_t red[kThreads / 64];
  // positive side: bit patterns p in [0, 0x7F800000), each against p + 1
  constexpr uint32_t kPos = kGeluKeyPosInf;
  // negative side: -0 ... -FLT_MAX, bit patterns 0x80000000 + [0, 0x7F800000)
  const uint32_t per = (kPos + uint32_t(kPremiseWgs) * kThreads - 1) / (uint32_t(kPremiseWgs) * kThreads);
  const uint32_t t0 = (uint32_t(blockIdx.x) * kThreads + threadIdx.x) * per;
  uint32_t viol = 0, tmax = 0;
  if (t0 < kPos) {
    float prev = gelu_f32(__uint_as_float(t0));
    for (uint32_t k = 0; k < per && t0 + k < kPos; ++k) {
      const uint32_t p = t0 + k;
      const float next = gelu_f32(__uint_as_float(p + 1));
      // a decrease, or a NaN anywhere on the way to +inf, fails the premise
      viol += (next < prev || next != next || prev != prev) ? 1u : 0u;
      prev = next;
      tmax = umax(tmax, absbits(gelu_f32(__uint_as_float(0x80000000u | p))));
    }
  }
  viol = block_umax_nt<kThreads>(viol, red);  // any violation (the count is not needed)
  __syncthreads();
  tmax = block_umax_nt<kThreads>(tmax, red);
  if (threadIdx.x == 0) {
    g_gelu_premise.wg_viol[blockIdx.x] = viol;
    g_gelu_premise.wg_t[blockIdx.x] = tmax;
  }
}

__global__ __launch_bounds__(kThreads) void gelu_premise_finalize_kernel() {
  __shared__ uint32_t red[kThreads / 64];
  uint32_t v = 0, t = 0;
  for (int i = threadIdx.x; i < kPremiseWgs; i += kThreads) {
    v = umax(v, g_gelu_premise.wg_viol[i]);
    t = umax(t, g_gelu_premise.wg_t[i]);
  }
  v = block_umax_nt<kThreads>(v, red);
  __syncthreads();
  t = block_umax_nt<kThreads>(t, red);
  if (threadIdx.x == 0) {
    g_gelu_premise.violations = v;
    g_gelu_premise.t_bits = t;
    __hip_atomic_store(&g_gelu_premise.done, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// The GELU amax rule on the keys of h's producer (keys[2 i], keys[2 i + 1],
// i < n_keys), then the partial maxima of |gelu(h)| for the quantising
// pass, in one launch.  Every workgroup reduces the keys (2 * n_keys words,
// L2 hits) to the same decision.  When the rule applies, workgroup 0 writes
// the amax it gives to part[0] and the others 0 (no pass over h); otherwise
// each workgroup takes its grid-stride share of h.  Workgroup 0 also
// records the decision in rule[0] (1: applied) and rule[1] (its amax bits).
__global__ __launch_bounds__(kGeluThreads) void gelu_amax_rule_kernel(
    const uint32_t* __restrict__ keys, int n_keys, const float* __restrict__ h, int64_t n,
    uint32_t* __restrict__ rule, uint32_t* __restrict__ part) {
  __shared__ uint32_t red[kGeluThreads / 64];
  __shared__ uint32_t red2[kGeluThreads / 64];
  uint32_t imax_biased = 0, umx = 0;  // int max kept as bits ^ 0x80000000 (unsigned order)
  for (int i = threadIdx.x; i < n_keys; i += kGeluThreads) {
    imax_biased = umax(imax_biased, keys[2 * i] ^ 0x80000000u);
    umx = umax(umx, keys[2 * i + 1]);
  }
  imax_biased = block_umax_nt<kGeluThreads>(imax_biased, red);
  umx = block_umax_nt<kGeluThreads>(umx, red2);
  // thread 0 decides and hands the decision to the workgroup through LDS
  // (its acquire load of the premise flag invalidates caches: one per
  // workgroup, not one per thread)
  __shared__ uint32_t dec[2];
  if (threadIdx.x == 0) {
    const uint32_t imax = imax_biased ^ 0x80000000u;
    // the premise check ran on this device (agent scope)
    const bool premises =
        __hip_atomic_load(&g_gelu_premise.done, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT) ==
            1u &&
        __hip_atomic_load(&g_gelu_premise.violations, __ATOMIC_RELAXED,
                          __HIP_MEMORY_SCOPE_AGENT) == 0u;
    bool ok = false;
    uint32_t abits = 0;
    if (premises && umx < kGeluKeyNegNanInf && int32_t(imax) >= 0 && imax <= kGeluKeyPosInf) {
      abits = absbits(gelu_f32(__uint_as_float(imax)));
      ok = abits >= __hip_atomic_load(&g_gelu_premise.t_bits, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT);
    }
    dec[0] = ok ? 1u : 0u;
    dec[1] = abits;
    if (blockIdx.x == 0) {
      rule[0] = dec[0];
      rule[1] = abits;
    }
  }
  __syncthreads();
  const bool ok = dec[0] != 0u;
  const uint32_t abits = dec[1];
  if (ok) {
    if (threadIdx.x == 0) part[blockIdx.x] = blockIdx.x == 0 ? abits : 0u;
    return;
  }
  uint32_t m = 0;
  const int64_t nvec = n >> 3;
  const int64_t stride = int64_t(gridDim.x) * kGeluThreads;
  for (int64_t i = int64_t(blockIdx.x) * kGeluThreads + threadIdx.x; i < nvec; i += stride) {
    float v[8];
    load8(h + i * 8, v);
#pragma unroll
    for (int j = 0; j < 8; ++j) m = umax(m, absbits(gelu_f32(v[j])));
  }
  for (int64_t t = nvec * 8 + int64_t(blockIdx.x) * kGeluThreads + threadIdx.x; t < n;
       t += stride)
    m = umax(m, absbits(gelu_f32(h[t])));
  __syncthreads();  // red is reused
  m = block_umax_nt<kGeluThreads>(m, red);
  if (threadIdx.x == 0) part[blockIdx.x] = m;
}

// out[c] = sum over row groups of cs_part[rg, c] (rg < rg_count): a workgroup owns 32
// columns with 8 row lanes, each lane summing every 8th row group with four
// independent loads in flight, then the lanes meet in LDS (fixed order).
__global__ __launch_bounds__(kThreads) void colsum_finalize_kernel(const float* __restrict__ cs_part,
                                                                   int rg_count, int64_t cols,
                                                                   float* __restrict__ out) {
  __shared__ float red[8][33];
  const int lc = threadIdx.x & 31, lr = threadIdx.x >> 5;
  const int64_t c = int64_t(blockIdx.x) * 32 + lc;
  float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
  if (c < cols) {
    int r = lr;
    for (; r + 24 < rg_count; r += 32) {
      s0 += cs_part[int64_t(r) * cols + c];
      s1 += cs_part[int64_t(r + 8) * cols + c];
      s2 += cs_part[int64_t(r + 16) * cols + c];
      s3 += cs_part[int64_t(r + 24) * cols + c];
    }
    for (; r < rg_count; r += 8) s0 += cs_part[int64_t(r) * cols + c];
  }
  red[lr][lc] = (s0 + s1) + (s2 + s3);
  __syncthreads();
  if (lr == 0 && c < cols) {
    float t = red[0][lc];
#pragma unroll
    for (int k = 1; k < 8; ++k) t += red[k][lc];
    out[c] = t;
  }
}

// q = RNE(clamp(x * scale)), flat, two vectors in flight per thread.
template <typename InT, int FMT>
__global__ __launch_bounds__(kThreads) void quant_flat_kernel(
    const InT* __restrict__ x, int64_t n, const uint32_t* __restrict__ part, int g, int bf16_rule,
    const float* __restrict__ scale_in, uint8_t* __restrict__ q, float* scale_out, float* inv_out) {
  __shared__ uint32_t red[kThreads / 64];
  const float mx = FMT == TCFP_FP8_E5M2 ? kE5M2Max : kE4M3Max;
  const float s = consumer_scale(scale_in, part, g, bf16_rule != 0, mx, scale_out, inv_out, red);
  const int64_t nvec = n >> 3;
  const int64_t stride = int64_t(gridDim.x) * kThreads;
  int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  for (; i + stride < nvec; i += 2 * stride) {
    float v[2][8];
    load8(x + i * 8, v[0]);
    load8(x + (i + stride) * 8, v[1]);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
#pragma unroll
      for (int j = 0; j < 8; ++j) v[u][j] = clampf(v[u][j] * s, mx);
      *reinterpret_cast<uint2*>(q + (i + u * stride) * 8) = encode8<FMT>(v[u]);
    }
  }
  for (; i < nvec; i += stride) {
    float v[8];
    load8(x + i * 8, v);
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = clampf(v[j] * s, mx);
    *reinterpret_cast<uint2*>(q + i * 8) = encode8<FMT>(v);
  }
  for (int64_t t = nvec * 8 + int64_t(blockIdx.x) * kThreads + threadIdx.x; t < n; t += stride)
    q[t] = uint8_t(encode1<FMT>(clampf(load1(x + t) * s, mx)));
}

// ---- 128 x 128 tiles with a transposed copy ------------------------------
// A workgroup quantises a 128 x 128 tile with 16-byte loads (a tile row is
// read by 32 (fp32) or 16 (bf16) consecutive lanes), stores the codes row by
// row, keeps them in LDS as 32 words per row, and writes the transposed
// tile: each lane gathers 16 rows of one word column, transposes the 4 x 4
// byte blocks in registers and stores 16-byte runs; 8 consecutive lanes
// cover one 128-byte output row segment.  Requires cols % 8 == 0, so every
// vector lies inside one row.
constexpr int kTile = 128;
constexpr int kTilePitch = kTile / 4 + 1;  // words per LDS row (+1 against bank conflicts)

struct TileGeom {
  int64_t r0, c0;
  int tiles_c;
  TCFP_DEV TileGeom(int64_t cols) : TileGeom(cols, int(blockIdx.x)) {}
  TCFP_DEV TileGeom(int64_t cols, int tile) {
    tiles_c = int((cols + kTile - 1) / kTile);
    r0 = int64_t(tile / tiles_c) * kTile;
    c0 = int64_t(tile % tiles_c) * kTile;
  }
};

// 16 tile rows of word column c4 -> 4 output columns of 16 bytes each.
TCFP_DEV void gather_transpose(const uint32_t* tile, int rc, int c4, uint4 out[4]) {
  uint32_t w[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) w[j] = tile[(rc * 16 + j) * kTilePitch + c4];
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    uint32_t o[4];
#pragma unroll
    for (int qd = 0; qd < 4; ++qd) {
      const int sh = 8 * b;
      o[qd] = ((w[4 * qd] >> sh) & 0xFFu) | (((w[4 * qd + 1] >> sh) & 0xFFu) << 8) |
              (((w[4 * qd + 2] >> sh) & 0xFFu) << 16) | (((w[4 * qd + 3] >> sh) & 0xFFu) << 24);
    }
    out[b] = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// Writes the transposed tile held in `tile` to dst [cols, rows]; `tid` in
// [0, 256) selects the 16-row x 4-column block this thread moves.
TCFP_DEV void store_transposed(const uint32_t* tile, const TileGeom& tg, int64_t rows,
                               int64_t cols, uint8_t* __restrict__ dst, int tid) {
  const int c4 = tid >> 3, rc = tid & 7;
  uint4 out[4];
  gather_transpose(tile, rc, c4, out);
  const int64_t r = tg.r0 + rc * 16;
  const bool fast = (rows % 16 == 0) && (r + 16 <= rows);
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const int64_t c = tg.c0 + c4 * 4 + b;
    if (c >= cols) continue;
    uint8_t* o = dst + c * rows + r;
    if (fast) {
      *reinterpret_cast<uint4*>(o) = out[b];
    } else {
      const uint32_t wd[4] = {out[b].x, out[b].y, out[b].z, out[b].w};
#pragma unroll
      for (int j = 0; j < 16; ++j)
        if (r + j < rows) o[j] = uint8_t(wd[j >> 2] >> (8 * (j & 3)));
    }
  }
}

template <typename InT>
struct TileLoad {
  static constexpr int VEC = 16 / int(sizeof(InT));  // elements per 16-byte load
  static constexpr int TPR = kTile / VEC;             // lanes per tile row
  static constexpr int RPI = kThreads / TPR;          // tile rows per pass
};

// loadvec with the non-temporal hint, for a pass that is its input's last
// reader: the streamed input then does not displace, in L2 and the Infinity
// Cache, the codes the next GEMM reads (C4 training step, one process:
// 0.851 -> 0.826 ms with the transposing pass's loads and the GELU
// derivative factors' stores streamed).
typedef float f32x4_nt __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_nt __attribute__((ext_vector_type(4)));
template <typename InT>
TCFP_DEV void loadvec_nt(const InT* p, float* v);
template <>
TCFP_DEV void loadvec_nt<float>(const float* p, float* v) {
  const f32x4_nt a = __builtin_nontemporal_load(reinterpret_cast<const f32x4_nt*>(p));
  v[0] = a[0]; v[1] = a[1]; v[2] = a[2]; v[3] = a[3];
}
template <>
TCFP_DEV void loadvec_nt<uint16_t>(const uint16_t* p, float* v) {
  const u32x4_nt a = __builtin_nontemporal_load(reinterpret_cast<const u32x4_nt*>(p));
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = __uint_as_float(a[i] << 16);
    v[2 * i + 1] = __uint_as_float(a[i] & 0xFFFF0000u);
  }
}
template <typename InT>
TCFP_DEV void loadvec(const InT* p, float* v);
template <>
TCFP_DEV void loadvec<float>(const float* p, float* v) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
}
template <>
TCFP_DEV void loadvec<uint16_t>(const uint16_t* p, float* v) { load8(p, v); }

// GELU_IN: the tile holds h and the pass quantises gelu(h), recomputed
// here (a producer wrote h and the partial maxima of |gelu(h)|); act_out
// and dg_out, when not null, receive gelu(h) and its derivative factor.
// COLSUM: the pass also writes the column sums of the values it quantises
// (before scaling) per 64-row group to cs_part[group, col], in the order
// of kColGroup's definition (rows past the end count as +0).  The tile's
// row lanes hold rows tr = pass * RPI + lane: the folds over row distances
// of RPI and more stay in a lane's registers, the rest meet in LDS.
// qt may be null (no transposed copy), and so may q when qt is not (only
// the transposed copy is written).
// (body: tile `bid`; nbk unused)
template <typename InT, int FMT, bool GELU_IN = false, bool COLSUM = false>
TCFP_DEV void quant_t_body(
    const InT* __restrict__ x, int64_t rows, int64_t cols, const uint32_t* __restrict__ part,
    int g, int bf16_rule, const float* __restrict__ scale_in, uint8_t* __restrict__ q,
    uint8_t* __restrict__ qt, float* scale_out, float* inv_out,
    float* __restrict__ cs_part, float* __restrict__ act_out,
    float* __restrict__ dg_out, const int bid, const int nbk, uint32_t* red, uint32_t* tile,
    float* csum) {
  using TL = TileLoad<InT>;
  constexpr int VEC = TL::VEC;
  // passes per half row group; the tile's two row groups, RPI row lanes each
  constexpr int PH = kColHalf / TL::RPI;
  static_assert(PH >= 1 && kTile == 2 * kColGroup, "row lanes per pass vs. row groups");
  const float mx = FMT == TCFP_FP8_E5M2 ? kE5M2Max : kE4M3Max;
  const float s = consumer_scale(scale_in, part, g, bf16_rule != 0, mx, scale_out, inv_out, red, bid);
  const TileGeom tg(cols, bid);
  const int tc = (threadIdx.x % TL::TPR) * VEC;
  const int rl = threadIdx.x / TL::TPR;
  const int64_t c = tg.c0 + tc;
  float ys[COLSUM ? PH : 1][VEC];  // x[l] + x[l + 32] of this lane's rows l of the group
#pragma unroll
  for (int it = 0; it < kTile / TL::RPI; ++it) {
    const int tr = it * TL::RPI + rl;
    const int64_t r = tg.r0 + tr;
    const bool valid = r < rows && c < cols;
    float v[VEC];
    if (valid) {
      loadvec_nt<InT>(x + r * cols + c, v);  // (the op's last read of x)
      if constexpr (GELU_IN) {
        if (dg_out) {
          float d[VEC];
#pragma unroll
          for (int j = 0; j < VEC; ++j) gelu_and_deriv(v[j], v[j], d[j]);
          // (read back only by the backward's dgrad, long after)
          const f32x4_nt dv = {d[0], d[1], d[2], d[3]};
          __builtin_nontemporal_store(dv, reinterpret_cast<f32x4_nt*>(dg_out + r * cols + c));
        } else {
#pragma unroll
          for (int j = 0; j < VEC; ++j) v[j] = gelu_f32(v[j]);
        }
        if (act_out)
          *reinterpret_cast<float4*>(act_out + r * cols + c) = make_float4(v[0], v[1], v[2], v[3]);
      }
    } else {
#pragma unroll
      for (int j = 0; j < VEC; ++j) v[j] = 0.0f;
    }
    if constexpr (COLSUM) {
      const int pg = it % (2 * PH);
      if (pg < PH) {
#pragma unroll
        for (int j = 0; j < VEC; ++j) ys[pg][j] = v[j];
      } else {
#pragma unroll
        for (int j = 0; j < VEC; ++j) ys[pg - PH][j] += v[j];
      }
      if (pg == 2 * PH - 1) {
        // folds over row distances 16 ... RPI (passes PH / 2 ... 1 apart)
#pragma unroll
        for (int d = PH / 2; d >= 1; d /= 2)
#pragma unroll
          for (int p = 0; p < d; ++p)
#pragma unroll
            for (int j = 0; j < VEC; ++j) ys[p][j] += ys[p + d][j];
        const int grp = it / (2 * PH);
#pragma unroll
        for (int j = 0; j < VEC; ++j) csum[(grp * TL::RPI + rl) * kTile + tc + j] = ys[0][j];
      }
    }
#pragma unroll
    for (int j = 0; j < VEC; ++j) v[j] = clampf(v[j] * s, mx);
    uint32_t wd[VEC / 4];
#pragma unroll
    for (int j = 0; j < VEC; j += 4) wd[j / 4] = encode4<FMT>(v[j], v[j + 1], v[j + 2], v[j + 3]);
    if (valid && q) {
      if constexpr (VEC == 4) *reinterpret_cast<uint32_t*>(q + r * cols + c) = wd[0];
      else *reinterpret_cast<uint2*>(q + r * cols + c) = make_uint2(wd[0], wd[1]);
    }
    if (qt) {
#pragma unroll
      for (int j = 0; j < VEC / 4; ++j) tile[tr * kTilePitch + tc / 4 + j] = wd[j];
    }
  }
  __syncthreads();
  if constexpr (COLSUM) {
    // the folds over row distances RPI / 2 ... 1: one (group, column) per thread
    static_assert(kThreads == 2 * kTile, "one thread per group column");
    const int grp = threadIdx.x / kTile, cl = threadIdx.x % kTile;
    float w[TL::RPI];
#pragma unroll
    for (int k = 0; k < TL::RPI; ++k) w[k] = csum[(grp * TL::RPI + k) * kTile + cl];
#pragma unroll
    for (int d = TL::RPI / 2; d >= 1; d /= 2)
#pragma unroll
      for (int k = 0; k < d; ++k) w[k] += w[k + d];
    const int64_t cc = tg.c0 + cl, r = tg.r0 + grp * kColGroup;
    if (cc < cols && r < rows) cs_part[(r / kColGroup) * cols + cc] = w[0];
  }
  if (qt) store_transposed(tile, tg, rows, cols, qt, threadIdx.x);
}

template <typename InT, int FMT, bool GELU_IN = false, bool COLSUM = false>
__global__ __launch_bounds__(kThreads) void quant_t_kernel(
    const InT* __restrict__ x, int64_t rows, int64_t cols, const uint32_t* __restrict__ part,
    int g, int bf16_rule, const float* __restrict__ scale_in, uint8_t* __restrict__ q,
    uint8_t* __restrict__ qt, float* scale_out, float* inv_out,
    float* __restrict__ cs_part = nullptr, float* __restrict__ act_out = nullptr,
    float* __restrict__ dg_out = nullptr) {
  __shared__ uint32_t red[kThreads / 64];
  __shared__ uint32_t tile[kTile * kTilePitch];
  __shared__ float csum[COLSUM ? 2 * TileLoad<InT>::RPI * kTile : 1];
  quant_t_body<InT, FMT, GELU_IN, COLSUM>(x, rows, cols, part, g, bf16_rule, scale_in, q, qt,
                                          scale_out, inv_out, cs_part, act_out, dg_out,
                                          int(blockIdx.x), int(gridDim.x), red, tile, csum);
}

// ===========================================================================
// Per-tensor dual quantisation (tcfp/nn/__init__.py:343-383)
// ===========================================================================
// Stochastic rounding of an already scaled and clamped value, following
// stochastic_round_to_fp8_e4m3 (tcfp/core.py:418-464) with torch's cast
// semantics (a candidate past 448 is the NaN code and is never selected).
TCFP_DEV uint32_t sr_per_tensor(float x, float u) {
  const uint32_t lo = f32_to_e4m3(x);
  const float lo_f = e4m3_to_f32(lo);
  if (x == lo_f) return lo;
  const float d = x > lo_f ? 1.0f : (x < lo_f ? -1.0f : 0.0f);
  uint32_t hi = f32_to_e4m3(lo_f + (d * 0.015625f) * 0.5f);
  if (e4m3_to_f32(hi) == lo_f) {
    const float abs_lo = fmaxf(fabsf(lo_f), 0.015625f);
    hi = f32_to_e4m3(lo_f + (d * abs_lo) * 0.25f);
  }
  const float hi_f = e4m3_to_f32(hi);
  float gap = fabsf(hi_f - lo_f);
  gap = (gap != gap) ? gap : fmaxf(gap, 1.4e-45f);
  float frac = fabsf(x - lo_f) / gap;
  frac = (frac != frac) ? frac : fminf(fmaxf(frac, 0.0f), 1.0f);
  return (u < frac) ? hi : lo;
}

// Stochastic W_hi codes (NF-aware scaling with stochastic=True) draw from
// their own Philox counters, 2^61 + e0 / 4 for the 4-element group at flat
// element e0 and 3 * 2^61 + t for a tail element t, apart from W_lo's
// (e0 / 4 and 2^62 + t): the two roundings are independent, and every pass
// that recomputes W_hi draws the same bits.
TCFP_DEV uint32_t hi_sr4(const float c[4], int64_t e0, uint32_t k0, uint32_t k1, uint32_t o0,
                         uint32_t o1) {
  const uint64_t ctr = (uint64_t(1) << 61) + (uint64_t(e0) >> 2);
  const u32x4 r = philox4x32_10({uint32_t(ctr), uint32_t(ctr >> 32), o0, o1}, k0, k1);
  return sr_per_tensor(c[0], u32_to_unit(r.x)) | (sr_per_tensor(c[1], u32_to_unit(r.y)) << 8) |
         (sr_per_tensor(c[2], u32_to_unit(r.z)) << 16) |
         (sr_per_tensor(c[3], u32_to_unit(r.w)) << 24);
}
TCFP_DEV uint32_t hi_sr1(float c, int64_t t, uint32_t k0, uint32_t k1, uint32_t o0, uint32_t o1) {
  const uint64_t ctr = (uint64_t(3) << 61) + uint64_t(t);
  const u32x4 r = philox4x32_10({uint32_t(ctr), uint32_t(ctr >> 32), o0, o1}, k0, k1);
  return sr_per_tensor(c, u32_to_unit(r.x));
}

// W_hi codes of the scaled, clamped values c[0..4) at flat element e0.
TCFP_DEV uint32_t hi_codes4(const float c[4], int64_t e0, bool sr, uint32_t k0, uint32_t k1,
                            uint32_t o0, uint32_t o1) {
  return sr ? hi_sr4(c, e0, k0, k1, o0, o1) : encode4<TCFP_FP8_E4M3>(c[0], c[1], c[2], c[3]);
}
TCFP_DEV uint32_t hi_code1(float c, int64_t t, bool sr, uint32_t k0, uint32_t k1, uint32_t o0,
                           uint32_t o1) {
  return sr ? hi_sr1(c, t, k0, k1, o0, o1) : encode1<TCFP_FP8_E4M3>(c);
}

// Pass 1 is amax_part_kernel<InT, HAS_EF, STATS> (partials a, and the sums
// of NF-aware scaling).

// The residual amax found among pass 1's candidates is the tensor's when
// every element left out provably has a smaller residual.  Those elements
// have |v| < amax * 4/7, so v * s_hi < 256 (1 + 2^-22) rounds to a code of
// at most 256 with an error of at most 8 (E4M3 spacing 16 in [128, 256);
// just above 256 the error is a few 2^-22), and the computed residual
// v - code * inv_hi stays below 8.00005 * inv_hi (the roundings of s_hi,
// inv_hi, the product and the difference add a few 2^-24).  So the candidates decide when their maximum exceeds
// 8.001 * inv_hi, no workgroup overflowed its region (its partial is
// 0xFFFFFFFF, a NaN, which no comparison passes) and the amax is finite.
TCFP_DEV bool cand_decisive(const uint32_t* pa, int ga, const uint32_t* pb2, int gc,
                            float inv_hi, uint32_t* red, uint32_t* red2) {
  const uint32_t a = __float_as_uint(reduce_parts(pa, ga, red));
  const float r = reduce_parts(pb2, gc, red2);
  return a < 0x7F800000u && r > 8.001f * inv_hi;
}

// Pass 2 over the candidates only: workgroup b reduces the residuals of
// the values in regions b, b + G, ... (the arithmetic of dualq_hi_kernel)
// into pb2[b], or 0xFFFFFFFF when one of them overflowed.  Workgroup 0
// publishes inv_hi and the W_hi target as dualq_hi_kernel does.
__global__ __launch_bounds__(kThreads) void cand_resid_kernel(
    const float* __restrict__ vals, const uint32_t* __restrict__ cnt, int cap,
    const uint32_t* __restrict__ pa, int ga, uint32_t* __restrict__ pb2, float* inv_hi_out,
    float* tgt_out) {
  __shared__ uint32_t red[kThreads / 64];
  __shared__ uint32_t red2[kThreads / 64];
  const float tgt = clamp_min_nan(reduce_parts(pa, ga, red), 1e-12f);
  float s_hi, inv_hi;
  scale_of(tgt, kE4M3Max, &s_hi, &inv_hi);
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    *inv_hi_out = inv_hi;
    *tgt_out = tgt;
  }
  bool ok = true;
  uint32_t m = 0;
  for (int b = blockIdx.x; b < ga; b += gridDim.x) {
    const uint32_t c = cnt[b];
    if (c > uint32_t(cap)) {
      ok = false;
      continue;
    }
    const float* v = vals + int64_t(b) * cap;
    for (uint32_t k = threadIdx.x; k < c; k += kThreads) {
      const float x = v[k];
      const uint32_t code = encode1<TCFP_FP8_E4M3>(clampf(x * s_hi, kE4M3Max));
      m = umax(m, absbits(x - e4m3_to_f32(code) * inv_hi));
    }
  }
  m = block_umax_all(m, red2);
  if (threadIdx.x == 0) pb2[blockIdx.x] = ok ? m : 0xFFFFFFFFu;
}

// Pass 2: W_hi codes and the partial max |residual| (partials b).
// (body: workgroup `bid` of `nbk`)
template <typename InT, bool HAS_EF>
TCFP_DEV void dualq_hi_body(
    const InT* __restrict__ w, const float* __restrict__ ef, int64_t n,
    const uint32_t* __restrict__ pa, int ga, uint8_t* __restrict__ hi, uint32_t* __restrict__ pb,
    float* inv_hi_out, Delayed dl, HiRule hr, uint32_t k0, uint32_t k1, uint32_t o0,
    uint32_t o1, float* tgt_out, const uint32_t* __restrict__ cand_b2, int gc, const int bid,
    const int nbk, uint32_t* red, uint32_t* red2, double* rd) {
  float s_hi, inv_hi;
  {
    const float tgt = hi_target(hr, pa, ga, red, rd);
    scale_of(dl.on ? delayed_amax(dl, tgt) : tgt, kE4M3Max, &s_hi, &inv_hi);
    if (bid == 0 && threadIdx.x == 0) {
      *inv_hi_out = inv_hi;
      *tgt_out = tgt;
    }
  }
  // after a candidate pass (which then leaves W_hi to pass 3): nothing to
  // do when the candidates decided the residual amax
  if (cand_b2 && cand_decisive(pa, ga, cand_b2, gc, inv_hi, red, red2)) return;
  const bool sr = hr.sr != 0;
  uint32_t m = 0;
  const int64_t nvec = n >> 3;
  const int64_t stride = int64_t(nbk) * kThreads;
  auto body = [&](const float v[8], int64_t i) {
    float c[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) c[j] = clampf(v[j] * s_hi, kE4M3Max);
    const uint2 code = sr ? make_uint2(hi_sr4(c, i * 8, k0, k1, o0, o1),
                                       hi_sr4(c + 4, i * 8 + 4, k0, k1, o0, o1))
                          : encode8<TCFP_FP8_E4M3>(c);
    if (hi) *reinterpret_cast<uint2*>(hi + i * 8) = code;
#pragma unroll
    for (int j = 0; j < 8; ++j) m = umax(m, absbits(v[j] - e4m3_to_f32(byte_of(code, j)) * inv_hi));
  };
  // The grid-stride slabs are visited last to first.  Pass 1 (same grid)
  // visited them first to last, and a vector is handled by the workgroup of
  // the same index in both passes, i.e. on the same XCD (workgroup b runs on
  // XCD b % 8), so the slabs pass 1 read last are still in that XCD's L2
  // when this pass starts; pass 3 goes first to last again.
  const int64_t i0 = int64_t(bid) * kThreads + threadIdx.x;
  int64_t i = i0 < nvec ? i0 + ((nvec - 1 - i0) / stride) * stride : -1;
  for (; i - stride >= i0; i -= 2 * stride) {
    float W[2][8], v[2][8];
    load_w8<InT, HAS_EF>(w, ef, i, W[0], v[0]);
    load_w8<InT, HAS_EF>(w, ef, i - stride, W[1], v[1]);
    body(v[0], i);
    body(v[1], i - stride);
  }
  for (; i >= i0; i -= stride) {
    float W[8], v[8];
    load_w8<InT, HAS_EF>(w, ef, i, W, v);
    body(v, i);
  }
  for (int64_t t = nvec * 8 + int64_t(bid) * kThreads + threadIdx.x; t < n; t += stride) {
    float v = load1(w + t);
    if constexpr (HAS_EF) v = v + ef[t];
    const uint32_t code = hi_code1(clampf(v * s_hi, kE4M3Max), t, sr, k0, k1, o0, o1);
    if (hi) hi[t] = uint8_t(code);
    m = umax(m, absbits(v - e4m3_to_f32(code) * inv_hi));
  }
  m = block_umax_all(m, red2);
  if (threadIdx.x == 0) pb[bid] = m;
}

template <typename InT, bool HAS_EF>
__global__ __launch_bounds__(kThreads) void dualq_hi_kernel(
    const InT* __restrict__ w, const float* __restrict__ ef, int64_t n,
    const uint32_t* __restrict__ pa, int ga, uint8_t* __restrict__ hi, uint32_t* __restrict__ pb,
    float* inv_hi_out, Delayed dl, HiRule hr, uint32_t k0, uint32_t k1, uint32_t o0,
    uint32_t o1, float* tgt_out, const uint32_t* __restrict__ cand_b2 = nullptr, int gc = 0) {
  __shared__ uint32_t red[kThreads / 64];
  __shared__ uint32_t red2[kThreads / 64];
  __shared__ double rd[2 * (kThreads / 64)];
  dualq_hi_body<InT, HAS_EF>(w, ef, n, pa, ga, hi, pb, inv_hi_out, dl, hr, k0, k1, o0, o1,
                             tgt_out, cand_b2, gc, int(blockIdx.x), int(gridDim.x), red, red2,
                             rd);
}

// W_lo codes of 4 consecutive elements starting at flat element `e0`
// (a multiple of 4).  SR draws Philox counter (e0 / 4) so that the random
// bits of an element depend only on its index.
template <bool SR>
TCFP_DEV uint32_t lo_codes4(const float x[4], int64_t e0, uint32_t k0, uint32_t k1, uint32_t o0,
                            uint32_t o1) {
  if constexpr (SR) {
    const uint64_t ctr = uint64_t(e0) >> 2;
    const u32x4 r = philox4x32_10({uint32_t(ctr), uint32_t(ctr >> 32), o0, o1}, k0, k1);
    return sr_per_tensor(x[0], u32_to_unit(r.x)) | (sr_per_tensor(x[1], u32_to_unit(r.y)) << 8) |
           (sr_per_tensor(x[2], u32_to_unit(r.z)) << 16) |
           (sr_per_tensor(x[3], u32_to_unit(r.w)) << 24);
  } else {
    return encode4<TCFP_FP8_E4M3>(x[0], x[1], x[2], x[3]);
  }
}

struct DualScales {
  float s_hi, inv_hi, s_lo, inv_lo;
};

// Pass-3 arithmetic for 4 elements: W_hi codes (recomputed exactly as in
// pass 2), W_lo codes, and the new error W - (deq(hi) + deq(lo)).
template <bool SR>
TCFP_DEV void dual_codes4(const float W[4], const float v[4], const DualScales& sc, int64_t e0,
                          bool srh, uint32_t k0, uint32_t k1, uint32_t o0, uint32_t o1,
                          uint32_t* hcode, uint32_t* lcode, float err[4]) {
  float c[4], dh[4], x[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) c[j] = clampf(v[j] * sc.s_hi, kE4M3Max);
  const uint32_t h = hi_codes4(c, e0, srh, k0, k1, o0, o1);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    dh[j] = e4m3_to_f32((h >> (8 * j)) & 0xFFu) * sc.inv_hi;
    x[j] = clampf((v[j] - dh[j]) * sc.s_lo, kE4M3Max);
  }
  const uint32_t l = lo_codes4<SR>(x, e0, k0, k1, o0, o1);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float dl = e4m3_to_f32((l >> (8 * j)) & 0xFFu) * sc.inv_lo;
    err[j] = W[j] - (dh[j] + dl);
  }
  *hcode = h;
  *lcode = l;
}

// `tgt_in`: the W_hi target the W_hi pass published (null: reduce it here).
// `pb2` (after a candidate pass): the gc candidates' residual partials,
// used in place of pb when they decide the residual amax.
TCFP_DEV DualScales dual_scales(const HiRule& hr, const float* tgt_in, const uint32_t* pa, int ga,
                                const uint32_t* pb, int gb, float* inv_lo_out, uint32_t* red,
                                uint32_t* red2, double* rd, const uint32_t* pb2 = nullptr,
                                int gc = 0, int bid = -1) {
  DualScales sc;
  scale_of(tgt_in ? *tgt_in : hi_target(hr, pa, ga, red, rd), kE4M3Max, &sc.s_hi, &sc.inv_hi);
  if (pb2 && cand_decisive(pa, ga, pb2, gc, sc.inv_hi, red, red2)) {
    pb = pb2;
    gb = gc;
  }
  sc.s_lo = consumer_scale(nullptr, pb, gb, false, kE4M3Max, nullptr, inv_lo_out, red2, bid);
  sc.inv_lo = __fdiv_rn(1.0f, sc.s_lo);
  return sc;
}

// Pass-3 scales under delayed scaling: W_hi from the EMA of the amax; W_lo
// from the measured residual amax on validation steps (updating the
// amax_lo / amax_hi ratio EMA, tcfp/core.py:374-393) or, otherwise, from
// the predicted one (delayed * ratio, or delayed / 8 before any ratio,
// :358-372).  Workgroup 0 writes both inverse scales and the new state.
TCFP_DEV DualScales dual_scales_delayed(const Delayed& d, const HiRule& hr, const float* tgt_in,
                                        const uint32_t* pa, int ga, const uint32_t* pb, int gb,
                                        float* inv_hi_out, float* inv_lo_out, uint32_t* red,
                                        uint32_t* red2, double* rd, int bid = -1) {
  DualScales sc;
  const float del = delayed_amax(d, tgt_in ? *tgt_in : hi_target(hr, pa, ga, red, rd));
  scale_of(del, kE4M3Max, &sc.s_hi, &sc.inv_hi);
  float lo_amax, ratio = 0.0f;
  if (d.validate) {
    lo_amax = clamp_min_nan(reduce_parts(pb, gb, red2), 1e-12f);
    const float r = __fdiv_rn(lo_amax, clamp_min_nan(del, 1e-12f));
    ratio = d.ratio_prev ? ema_f32(*d.ratio_prev, r, d.a, d.b) : r;
  } else {
    lo_amax = clamp_min_nan(d.ratio_prev ? __fmul_rn(del, *d.ratio_prev) : __fdiv_rn(del, 8.0f),
                            1e-12f);
  }
  scale_of(lo_amax, kE4M3Max, &sc.s_lo, &sc.inv_lo);
  if ((bid < 0 ? int(blockIdx.x) : bid) == 0 && threadIdx.x == 0) {
    *inv_hi_out = sc.inv_hi;
    *inv_lo_out = sc.inv_lo;
    *d.amax_out = del;
    if (d.validate) *d.ratio_out = ratio;
  }
  return sc;
}

// Pass 3 (flat): W_lo codes (RNE or SR) and, optionally, the new error in place.
template <typename InT, bool HAS_EF, bool UPDATE, bool SR>
__global__ __launch_bounds__(kThreads) void dualq_lo_kernel(
    const InT* __restrict__ w, float* __restrict__ ef, int64_t n, const uint32_t* __restrict__ pa,
    int ga, const uint32_t* __restrict__ pb, int gb, uint8_t* __restrict__ lo, float* inv_lo_out,
    uint32_t k0, uint32_t k1, uint32_t off0, uint32_t off1, Delayed dl, float* inv_hi_out,
    uint8_t* __restrict__ hi, HiRule hr, const float* tgt_in, const uint32_t* pb2, int gc) {
  __shared__ uint32_t red[kThreads / 64];
  __shared__ uint32_t red2[kThreads / 64];
  __shared__ double rd[2 * (kThreads / 64)];
  const DualScales sc =
      dl.on ? dual_scales_delayed(dl, hr, tgt_in, pa, ga, pb, gb, inv_hi_out, inv_lo_out, red,
                                  red2, rd)
            : dual_scales(hr, tgt_in, pa, ga, pb, gb, inv_lo_out, red, red2, rd, pb2, gc);
  const bool srh = hr.sr != 0;
  const int64_t nvec = n >> 3;
  const int64_t stride = int64_t(gridDim.x) * kThreads;
  auto body = [&](const float W[8], const float v[8], int64_t i) {
    uint32_t hc[2], lc[2];
    float e[8];
    dual_codes4<SR>(W, v, sc, i * 8, srh, k0, k1, off0, off1, &hc[0], &lc[0], e);
    dual_codes4<SR>(W + 4, v + 4, sc, i * 8 + 4, srh, k0, k1, off0, off1, &hc[1], &lc[1], e + 4);
    *reinterpret_cast<uint2*>(lo + i * 8) = make_uint2(lc[0], lc[1]);
    // W_hi codes when no earlier pass wrote them
    if (hi) *reinterpret_cast<uint2*>(hi + i * 8) = make_uint2(hc[0], hc[1]);
    if constexpr (HAS_EF && UPDATE) store8(ef + i * 8, e);
  };
  int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  for (; i + stride < nvec; i += 2 * stride) {
    float W[2][8], v[2][8];
    load_w8<InT, HAS_EF>(w, ef, i, W[0], v[0]);
    load_w8<InT, HAS_EF>(w, ef, i + stride, W[1], v[1]);
    body(W[0], v[0], i);
    body(W[1], v[1], i + stride);
  }
  for (; i < nvec; i += stride) {
    float W[8], v[8];
    load_w8<InT, HAS_EF>(w, ef, i, W, v);
    body(W, v, i);
  }
  for (int64_t t = nvec * 8 + int64_t(blockIdx.x) * kThreads + threadIdx.x; t < n; t += stride) {
    const float W = load1(w + t);
    float v = W;
    if constexpr (HAS_EF) v = W + ef[t];
    const uint32_t hcode = hi_code1(clampf(v * sc.s_hi, kE4M3Max), t, srh, k0, k1, off0, off1);
    if (hi) hi[t] = uint8_t(hcode);
    const float dh = e4m3_to_f32(hcode) * sc.inv_hi;
    const float x = clampf((v - dh) * sc.s_lo, kE4M3Max);
    uint32_t lcode;
    if constexpr (SR) {
      const uint64_t ctr = (uint64_t(1) << 62) + uint64_t(t);
      u32x4 r = philox4x32_10({uint32_t(ctr), uint32_t(ctr >> 32), off0, off1}, k0, k1);
      lcode = sr_per_tensor(x, u32_to_unit(r.x));
    } else {
      lcode = encode1<TCFP_FP8_E4M3>(x);
    }
    lo[t] = uint8_t(lcode);
    if constexpr (HAS_EF && UPDATE) ef[t] = W - (dh + e4m3_to_f32(lcode) * sc.inv_lo);
  }
}

// Pass 3 (tiled, cols % 8 == 0): as dualq_lo_kernel on 128 x 128 tiles, and
// also writes the transposed W_hi and W_lo codes (the dgrad operands).
// (body: tile `bid`; nbk unused)
template <typename InT, bool HAS_EF, bool UPDATE, bool SR>
TCFP_DEV void dualq_lo_t_body(
    const InT* __restrict__ w, float* __restrict__ ef, int64_t rows, int64_t cols,
    const uint32_t* __restrict__ pa, int ga, const uint32_t* __restrict__ pb, int gb,
    uint8_t* __restrict__ lo, float* inv_lo_out, uint8_t* __restrict__ hi_t,
    uint8_t* __restrict__ lo_t, uint32_t k0, uint32_t k1, uint32_t off0, uint32_t off1,
    Delayed dl, float* inv_hi_out, uint8_t* __restrict__ hi, HiRule hr, const float* tgt_in,
    const uint32_t* pb2, int gc, const int bid, const int nbk, uint32_t* red, uint32_t* red2,
    double* rd, uint32_t* tile_h, uint32_t* tile_l) {
  using TL = TileLoad<InT>;
  constexpr int VEC = TL::VEC;
  const DualScales sc =
      dl.on ? dual_scales_delayed(dl, hr, tgt_in, pa, ga, pb, gb, inv_hi_out, inv_lo_out, red,
                                  red2, rd, bid)
            : dual_scales(hr, tgt_in, pa, ga, pb, gb, inv_lo_out, red, red2, rd, pb2, gc, bid);
  const bool srh = hr.sr != 0;
  const TileGeom tg(cols, bid);
  const int tc = (threadIdx.x % TL::TPR) * VEC;
  const int64_t c = tg.c0 + tc;
#pragma unroll 2
  for (int it = 0; it < kTile / TL::RPI; ++it) {
    const int tr = it * TL::RPI + threadIdx.x / TL::TPR;
    const int64_t r = tg.r0 + tr;
    const bool valid = r < rows && c < cols;
    const int64_t off = r * cols + c;
    float W[VEC], v[VEC];
    if (valid) {
      loadvec<InT>(w + off, W);
    } else {
#pragma unroll
      for (int j = 0; j < VEC; ++j) W[j] = 0.0f;
    }
    if constexpr (HAS_EF) {
      float e[VEC];
      if (valid) {
#pragma unroll
        for (int j = 0; j < VEC; j += 4) {
          const float4 a = *reinterpret_cast<const float4*>(ef + off + j);
          e[j] = a.x; e[j + 1] = a.y; e[j + 2] = a.z; e[j + 3] = a.w;
        }
      } else {
#pragma unroll
        for (int j = 0; j < VEC; ++j) e[j] = 0.0f;
      }
#pragma unroll
      for (int j = 0; j < VEC; ++j) v[j] = W[j] + e[j];
    } else {
#pragma unroll
      for (int j = 0; j < VEC; ++j) v[j] = W[j];
    }
    uint32_t hc[VEC / 4], lc[VEC / 4];
    float err[VEC];
#pragma unroll
    for (int j = 0; j < VEC; j += 4)
      dual_codes4<SR>(W + j, v + j, sc, off + j, srh, k0, k1, off0, off1, &hc[j / 4],
                      &lc[j / 4], err + j);
    if (valid) {
      if constexpr (VEC == 4) *reinterpret_cast<uint32_t*>(lo + off) = lc[0];
      else *reinterpret_cast<uint2*>(lo + off) = make_uint2(lc[0], lc[1]);
      if (hi) {  // W_hi codes when no earlier pass wrote them
        if constexpr (VEC == 4) *reinterpret_cast<uint32_t*>(hi + off) = hc[0];
        else *reinterpret_cast<uint2*>(hi + off) = make_uint2(hc[0], hc[1]);
      }
      if constexpr (HAS_EF && UPDATE) {
#pragma unroll
        for (int j = 0; j < VEC; j += 4)
          *reinterpret_cast<float4*>(ef + off + j) =
              make_float4(err[j], err[j + 1], err[j + 2], err[j + 3]);
      }
    }
#pragma unroll
    for (int j = 0; j < VEC / 4; ++j) {
      tile_h[tr * kTilePitch + tc / 4 + j] = hc[j];
      tile_l[tr * kTilePitch + tc / 4 + j] = lc[j];
    }
  }
  __syncthreads();
  if (hi_t) store_transposed(tile_h, tg, rows, cols, hi_t, threadIdx.x);
  if (lo_t) store_transposed(tile_l, tg, rows, cols, lo_t, threadIdx.x);
}

template <typename InT, bool HAS_EF, bool UPDATE, bool SR>
__global__ __launch_bounds__(kThreads) void dualq_lo_t_kernel(
    const InT* __restrict__ w, float* __restrict__ ef, int64_t rows, int64_t cols,
    const uint32_t* __restrict__ pa, int ga, const uint32_t* __restrict__ pb, int gb,
    uint8_t* __restrict__ lo, float* inv_lo_out, uint8_t* __restrict__ hi_t,
    uint8_t* __restrict__ lo_t, uint32_t k0, uint32_t k1, uint32_t off0, uint32_t off1,
    Delayed dl, float* inv_hi_out, uint8_t* __restrict__ hi, HiRule hr, const float* tgt_in,
    const uint32_t* pb2, int gc) {
  __shared__ uint32_t red[kThreads / 64];
  __shared__ uint32_t red2[kThreads / 64];
  __shared__ double rd[2 * (kThreads / 64)];
  __shared__ uint32_t tile_h[kTile * kTilePitch];
  __shared__ uint32_t tile_l[kTile * kTilePitch];
  dualq_lo_t_body<InT, HAS_EF, UPDATE, SR>(w, ef, rows, cols, pa, ga, pb, gb, lo, inv_lo_out,
                                           hi_t, lo_t, k0, k1, off0, off1, dl, inv_hi_out, hi,
                                           hr, tgt_in, pb2, gc, int(blockIdx.x),
                                           int(gridDim.x), red, red2, rd, tile_h, tile_l);
}
// ===========================================================================
// Per-tensor stochastic rounding (to_fp8_e4m3_sr, tcfp/core.py:109-134)
// ===========================================================================
// c = clamp(x * scale) with the per-tensor scale rule (or a given scale),
// then the stochastic_round_to_fp8_e4m3 rule (tcfp/core.py:418-464) on c:
// RNE candidate, its neighbour toward c, up with probability |c - lo| / gap.
// Element e of a 4-element group starting at flat index e0 draws word
// (e - e0) of Philox4x32-10 counter (e0 / 4, 0, offset); a tail element t
// (past the last 8-element vector) draws counter 2^62 + t.  The draw of an
// element depends on its index only, not on the launch shape.
template <typename InT>
__global__ __launch_bounds__(kThreads) void quant_sr_kernel(
    const InT* __restrict__ x, int64_t n, const uint32_t* __restrict__ part, int g, int bf16_rule,
    const float* __restrict__ scale_in, uint8_t* __restrict__ q, float* scale_out, float* inv_out,
    uint32_t k0, uint32_t k1, uint32_t o0, uint32_t o1) {
  __shared__ uint32_t red[kThreads / 64];
  const float s = consumer_scale(scale_in, part, g, bf16_rule != 0, kE4M3Max, scale_out, inv_out,
                                 red);
  const int64_t nvec = n >> 3;
  const int64_t stride = int64_t(gridDim.x) * kThreads;
  for (int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x; i < nvec; i += stride) {
    float v[8];
    load8(x + i * 8, v);
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = clampf(v[j] * s, kE4M3Max);
    const uint32_t c0 = lo_codes4<true>(v, i * 8, k0, k1, o0, o1);
    const uint32_t c1 = lo_codes4<true>(v + 4, i * 8 + 4, k0, k1, o0, o1);
    *reinterpret_cast<uint2*>(q + i * 8) = make_uint2(c0, c1);
  }
  for (int64_t t = nvec * 8 + int64_t(blockIdx.x) * kThreads + threadIdx.x; t < n; t += stride) {
    const float c = clampf(load1(x + t) * s, kE4M3Max);
    const uint64_t ctr = (uint64_t(1) << 62) + uint64_t(t);
    const u32x4 r = philox4x32_10({uint32_t(ctr), uint32_t(ctr >> 32), o0, o1}, k0, k1);
    q[t] = uint8_t(sr_per_tensor(c, u32_to_unit(r.x)));
  }
}

// ===========================================================================
// Power-of-two block scales (compute_block_scales, tcfp/core.py:221-252)
// ===========================================================================
// scale = 2^ceil(log2(max(amax, 1e-12) / fp8_max)) per run of `block`
// elements, every step rounded to the input dtype as torch's ops round it:
//   fp32: q = amax / fp8_max (IEEE), ceil(log2 q) by the exact integer rule
//         of a correctly rounded fp32 log2 (ceil_log2_f32), 2^e;
//   bf16: the 1e-12 bound and q rounded to bf16, log2 q evaluated in fp32
//         (an fp64 log2 rounded once) and rounded to bf16 -- that 8-bit
//         rounding can pull a value just above an integer down onto it --
//         then ceil, 2^e rounded to bf16.
// NaN propagates; q = 0 gives 0 and q = inf gives inf, as log2/exp2 do.
TCFP_DEV float pow2_of(float e) {
  if (e != e) return e;
  if (e >= 128.0f) return __uint_as_float(0x7F800000u);
  if (e < -149.0f) return 0.0f;
  return exp2i(int(e));
}

TCFP_DEV float block_scale_f32(float amax, float fmax) {
  if (amax != amax) return amax;
  const float q = __fdiv_rn(fmaxf(amax, 1e-12f), fmax);
  if (q != q || q == 0.0f || q == __uint_as_float(0x7F800000u)) return q;
  if (q >= 1.17549435e-38f) return pow2_of(float(ceil_log2_f32(q)));
  return pow2_of(ceilf(float(log2(double(q)))));  // subnormal quotient
}

TCFP_DEV float block_scale_bf16(float amax, float fmax) {
  if (amax != amax) return amax;
  const float q = round_bf16(__fdiv_rn(fmaxf(amax, round_bf16(1e-12f)), fmax));
  if (q != q || q == 0.0f || q == __uint_as_float(0x7F800000u)) return q;
  const float l = round_bf16(float(log2(double(q))));
  return round_bf16(pow2_of(ceilf(l)));
}

TCFP_DEV float abs_load(const float* p) { return fabsf(*p); }
TCFP_DEV float abs_load(const uint16_t* p) { return fabsf(bf16_to_f32(*p)); }
TCFP_DEV void store_scale(float* p, float v) { *p = v; }
TCFP_DEV void store_scale(uint16_t* p, float v) { *p = f32_to_bf16_rne(v); }

// One block per lane: a lane reads its `block` consecutive elements.
template <typename InT>
__global__ __launch_bounds__(kThreads) void block_scales_kernel(const InT* __restrict__ x,
                                                                int64_t nblocks, int block,
                                                                float fmax,
                                                                InT* __restrict__ out) {
  const int64_t stride = int64_t(gridDim.x) * kThreads;
  for (int64_t b = int64_t(blockIdx.x) * kThreads + threadIdx.x; b < nblocks; b += stride) {
    const InT* p = x + b * block;
    float m = 0.0f;
    for (int i = 0; i < block; ++i) m = nanmax(m, abs_load(p + i));
    if constexpr (sizeof(InT) == 4)
      store_scale(out + b, block_scale_f32(m, fmax));
    else
      store_scale(out + b, block_scale_bf16(m, fmax));
  }
}

// ===========================================================================
// Block quantisation (tcfp/kernels.py:205-275)
// ===========================================================================

// Segment geometry: one (row, K-block) segment of BS elements is read by
// L = BS / VEC lanes with one 16-byte load each; a 256-thread workgroup
// covers 256 / L consecutive rows of one K-block, so the int8 exponents of
// a workgroup ([K/bs, M] layout) are contiguous.
// (row group, K-block) of this workgroup in the block quantisers' grids.
//  kfast (a 1-D grid of row groups x kbs items): K-blocks fastest, and
//    workgroup b (dispatched to XCD b % 8) takes item (b % 8) * T/8 + b / 8:
//    each XCD walks its own contiguous run of whole row groups, so the
//    workgroups resident at once cover a few MB and the two halves of a
//    128-byte line (64-byte row pieces: bf16 at block 32) stay in one L2.
//    From 64 MB of input: 8192 x 16384 fp32 at block 64 ran 127 us against
//    205 us in row-group order.
//  otherwise (grid x = row group, y = K-block): row groups fastest, one
//    K-block of many rows at a time, ~1 us faster on 32 MB inputs.
TCFP_DEV void block_item(int64_t kbs64, bool kfast, uint32_t& rg, int64_t& kb) {
  if (kfast) {
    const uint32_t b = blockIdx.x, t = gridDim.x, kbs = uint32_t(kbs64);
    const uint32_t i = (t & 7u) == 0 ? (b & 7u) * (t >> 3) + (b >> 3) : b;
    rg = i / kbs;
    kb = i - rg * kbs;
  } else {
    rg = blockIdx.x;
    kb = blockIdx.y;
  }
}

// Inputs of at least this many bytes take the K-fastest order above.
constexpr int64_t kKFastBytes = int64_t(64) << 20;

template <typename InT, int BS, int V = 16 / int(sizeof(InT))>
struct Seg {
  static constexpr int VEC = V;
  static constexpr int L = BS / VEC;
  static constexpr int ROWS = kThreads / L;
};

template <typename InT>
TCFP_DEV void loadv(const InT* p, float* v);
template <>
TCFP_DEV void loadv<float>(const float* p, float* v) { loadvec_nt<float>(p, v); }
// (loadv / loadf / load_in serve the one-pass block quantisers, their
// input's last readers this step: streamed, C5 scale-up 8.48 -> 8.45 ms)
template <>
TCFP_DEV void loadv<uint16_t>(const uint16_t* p, float* v) { loadvec_nt<uint16_t>(p, v); }

template <int N>
TCFP_DEV void loadf(const float* p, float* v) {
#pragma unroll
  for (int i = 0; i < N; i += 4) loadvec_nt<float>(p + i, v + i);
}
template <int N>
TCFP_DEV void storef(float* p, const float* v) {
#pragma unroll
  for (int i = 0; i < N; i += 4)
    *reinterpret_cast<float4*>(p + i) = make_float4(v[i], v[i + 1], v[i + 2], v[i + 3]);
}

template <int N, int FMT>
TCFP_DEV void encodeN(const float* v, uint8_t* dst) {
  if constexpr (N == 4) {
#ifdef TCFP_SW_CVT
    *reinterpret_cast<uint32_t*>(dst) = sw4_fp8<FMT>(v[0], v[1], v[2], v[3]);
#else
    *reinterpret_cast<uint32_t*>(dst) = cvt4_fp8<FMT>(v[0], v[1], v[2], v[3]);
#endif
  } else {
    *reinterpret_cast<uint2*>(dst) = encode8<FMT>(v);
  }
}

template <int N, int FMT>
TCFP_DEV void encode_words(const float* v, uint32_t* words) {
#pragma unroll
  for (int i = 0; i < N; i += 4) {
#ifdef TCFP_SW_CVT
    words[i / 4] = sw4_fp8<FMT>(v[i], v[i + 1], v[i + 2], v[i + 3]);
#else
    words[i / 4] = cvt4_fp8<FMT>(v[i], v[i + 1], v[i + 2], v[i + 3]);
#endif
  }
}

template <int N>
TCFP_DEV void store_words(uint8_t* dst, const uint32_t* words) {
  if constexpr (N == 4) *reinterpret_cast<uint32_t*>(dst) = words[0];
  else if constexpr (N == 8) *reinterpret_cast<uint2*>(dst) = make_uint2(words[0], words[1]);
  else *reinterpret_cast<uint4*>(dst) = make_uint4(words[0], words[1], words[2], words[3]);
  static_assert(N == 4 || N == 8 || N == 16, "4, 8 or 16 codes");
}

TCFP_DEV uint32_t wbyte(const uint32_t* words, int j) { return (words[j >> 2] >> (8 * (j & 3))) & 0xFFu; }

// Block scale rules.  F32S == false: the reference's power-of-two exponent
// (int8 [K/bs, rows]).  F32S == true: to_fp8_e4m3's per-tensor rule
// (tcfp/core.py:99-106) applied to each block -- scale = FP8_MAX / amax with
// the reciprocal and the product rounded to the input dtype, codes
// RNE(clamp(x * scale)) -- storing the fp32 inverse scale 1 / scale
// ([K/bs, rows]), the block's dequantisation multiplier.
template <typename InT, int FMT, int BS, bool F32S>
__global__ __launch_bounds__(kThreads) void block_quant_kernel(const InT* __restrict__ x,
                                                               int64_t m, int64_t k,
                                                               uint8_t* __restrict__ q,
                                                               void* __restrict__ scales,
                                                               bool kfast) {
  using G = Seg<InT, BS>;
  constexpr int VEC = G::VEC;
  uint32_t rg;
  int64_t kb;
  block_item(k / BS, kfast, rg, kb);
  const int64_t row = int64_t(rg) * G::ROWS + threadIdx.x / G::L;
  const int li = threadIdx.x % G::L;
  const bool valid = row < m;
  const int64_t off = row * k + kb * BS + li * VEC;
  float v[VEC];
  if (valid) {
    loadv<InT>(x + off, v);
  } else {
#pragma unroll
    for (int j = 0; j < VEC; ++j) v[j] = 0.0f;
  }
  uint32_t a = 0;
#pragma unroll
  for (int j = 0; j < VEC; ++j) a = umax(a, absbits(v[j]));
  a = seg_umax<G::L>(a);
  const float mx = FMT == TCFP_FP8_E5M2 ? kE5M2Max : kE4M3Max;
  float mul, inv = 0.0f;
  int e = 0;
  if constexpr (F32S) {
    scale_from_amax(__uint_as_float(a), sizeof(InT) == 2, mx, &mul, &inv);
  } else {
    e = block_exponent(__uint_as_float(a), mx);
    mul = exp2i(-e);
  }
#pragma unroll
  for (int j = 0; j < VEC; ++j) v[j] = clampf(v[j] * mul, mx);
  if (valid) {
    encodeN<VEC, FMT>(v, q + off);
    if (li == 0) {
      if constexpr (F32S) static_cast<float*>(scales)[kb * m + row] = inv;
      else static_cast<int8_t*>(scales)[kb * m + row] = int8_t(e);
    }
  }
}

// Elements per lane of the dual kernel (each Philox call of the stochastic
// variants -- 8 x 16 random bits -- serves 8 of them): with stochastic
// rounding 8 (fp32) or 16 (bf16), otherwise one 16-byte load (4 fp32 or
// 8 bf16), or 8 fp32 for 32-element blocks.  Measured fastest on MI355X
// among 4/8/16 elements per lane, contiguous or in interleaved 16-byte
// chunks (SRR 16384 x 4096: 110 us at 8 fp32 against 116-182 us).
template <typename InT, int BS, bool SR>
using DualSeg = Seg<InT, BS, SR ? 16 / int(sizeof(InT)) * 2 : (BS == 32 ? 8 : 16 / int(sizeof(InT)))>;

template <typename InT, int N>
TCFP_DEV void load_in(const InT* p, float* v) {
  if constexpr (sizeof(InT) == 4) {
    loadf<N>(reinterpret_cast<const float*>(p), v);
  } else {
    static_assert(N % 8 == 0, "bf16 segments load 8 elements at a time");
#pragma unroll
    for (int i = 0; i < N; i += 8) loadvec_nt<uint16_t>(reinterpret_cast<const uint16_t*>(p) + i, v + i);
  }
}

// Block stochastic rounding (tcfp/kernels.py:398-423): the neighbour is
// found by a quarter-magnitude nudge under a saturating cast, and is taken
// with probability |diff| / gap.  The draw u = k * 2^-16 (k a 16-bit
// integer) is compared as u * gap < |diff|: u has 16 significant bits and
// gap, the distance between two E4M3 values no more than ~0.6 |rtn| apart,
// at most 5, so the product is exact and the test is the exact comparison
// u < |diff| / gap, with no division.  diff == 0 keeps rtn (the product is
// not below 0); gap == 0 (the nudge rounds back to rtn's value) keeps rtn;
// a NaN x keeps rtn (its own NaN code) since every comparison is false.
TCFP_DEV bool sr_take(float diff, float g, float u) { return g != 0.0f && u * g < fabsf(diff); }

TCFP_DEV uint32_t sr_block(float x, float u) {
  const uint32_t rtn = f32_to_e4m3(x, true);
  const float rtn_f = sw_e4m3_to_f32(rtn);
  const float diff = x - rtn_f;
  const float q = fmaxf(fabsf(rtn_f), 1e-12f) * 0.25f;
  const float nud = rtn_f + (diff >= 0.0f ? q : -q);
  const uint32_t other = f32_to_e4m3(clampf(nud, kE4M3Max), true);
  const float other_f = sw_e4m3_to_f32(other);
  return sr_take(diff, fabsf(other_f - rtn_f), u) ? other : rtn;
}

// sr_block on the hardware converts.  Both encodes see clamped inputs
// (|x| <= 448, the nudged value is clamped), where v_cvt_pk_fp8_f32 is the
// RNE encoder (bit-identical to the software one over every finite float in
// range, GPU self-test) and saturation never triggers; v_cvt_f32_fp8 decodes
// exactly.  tcfp_selftest_sr_block compares the two functions bit for bit.
TCFP_DEV uint32_t hw_e4m3(float x) {
  return uint32_t(__builtin_amdgcn_cvt_pk_fp8_f32(x, 0.0f, 0, false)) & 0xFFu;
}
TCFP_DEV float hw_e4m3_f32(uint32_t c) { return __builtin_amdgcn_cvt_f32_fp8(int(c), 0); }

TCFP_DEV uint32_t sr_block_hw(float x, float u) {
  const uint32_t rtn = hw_e4m3(x);
  const float rtn_f = hw_e4m3_f32(rtn);
  const float diff = x - rtn_f;
  const float q = fmaxf(fabsf(rtn_f), 1e-12f) * 0.25f;
  const float nud = rtn_f + (diff >= 0.0f ? q : -q);
  const uint32_t other = hw_e4m3(clampf(nud, kE4M3Max));
  const float other_f = hw_e4m3_f32(other);
  return sr_take(diff, fabsf(other_f - rtn_f), u) ? other : rtn;
}

// sr_block_hw on four values c[0..4) with packed converts (two values per
// encode or decode).  Value j draws the 16-bit field j of (r0, r1), low
// half first, as u = k * 2^-16.  Returns the four codes, value j in byte j.
// The nudged values are clamped with fmin/fmax: for a NaN c[j] the choice
// is rtn whatever the candidate is.
TCFP_DEV uint32_t sr_block_hw4(const float* c, uint32_t r0, uint32_t r1) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  const uint32_t rtn = cvt4_fp8<TCFP_FP8_E4M3>(c[0], c[1], c[2], c[3]);
  const f2 ra = __builtin_amdgcn_cvt_pk_f32_fp8(int(rtn), false);
  const f2 rb = __builtin_amdgcn_cvt_pk_f32_fp8(int(rtn), true);
  const float rf[4] = {ra[0], ra[1], rb[0], rb[1]};
  float diff[4], nud[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    diff[j] = c[j] - rf[j];
    // the nudge takes diff's sign (for diff == -0 too: the choice is rtn then)
    const float q = __builtin_copysignf(fmaxf(fabsf(rf[j]), 1e-12f) * 0.25f, diff[j]);
    nud[j] = fminf(fmaxf(rf[j] + q, -kE4M3Max), kE4M3Max);
  }
  const uint32_t oth = cvt4_fp8<TCFP_FP8_E4M3>(nud[0], nud[1], nud[2], nud[3]);
  const f2 oa = __builtin_amdgcn_cvt_pk_f32_fp8(int(oth), false);
  const f2 ob = __builtin_amdgcn_cvt_pk_f32_fp8(int(oth), true);
  const float of[4] = {oa[0], oa[1], ob[0], ob[1]};
  const uint32_t k[4] = {r0 & 0xFFFFu, r0 >> 16, r1 & 0xFFFFu, r1 >> 16};
  // sr_take without its gap == 0 guard: a zero gap means the candidate has
  // rtn's value, and then also rtn's code unless both are zeros, which
  // happens only with diff == 0 (an exact x), where the strict comparison
  // already keeps rtn.  (The self-test checks this form against sr_block,
  // guard included, on every float in range.)
  uint32_t mask = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float u = float(k[j]) * 1.52587890625e-05f;
    if (u * fabsf(of[j] - rf[j]) < fabsf(diff[j])) mask |= 0xFFu << (8 * j);
  }
  return (oth & mask) | (rtn & ~mask);
}

// Fused block dual quantisation + error update (tcfp/kernels.py:288-459 and
// :1867-1873).  The error buffer is read and rewritten by the same lane.
// With F32S the two components use the fp32 block rule above on the fp32
// values w + e and r (no zero-block sentinel: a zero residual gets the
// clamped 1e-12 amax and zero codes).
template <typename InT, int BS, bool HAS_EF, bool UPDATE, bool SR, bool F32S>
__global__ __launch_bounds__(kThreads) void block_dualq_kernel(
    const InT* __restrict__ w, float* __restrict__ ef, int64_t n, int64_t k,
    uint8_t* __restrict__ hi, uint8_t* __restrict__ lo, void* __restrict__ shi,
    void* __restrict__ slo, uint32_t k0, uint32_t k1, uint32_t off0, uint32_t off1, bool kfast) {
  using G = DualSeg<InT, BS, SR>;
  constexpr int VEC = G::VEC;
  uint32_t rg;
  int64_t kb;
  block_item(k / BS, kfast, rg, kb);
  const int64_t row = int64_t(rg) * G::ROWS + threadIdx.x / G::L;
  const int li = threadIdx.x % G::L;
  const bool valid = row < n;
  const int64_t off = row * k + kb * BS + li * VEC;
  float W[VEC], v[VEC];
  if (valid) {
    load_in<InT, VEC>(w + off, W);
  } else {
#pragma unroll
    for (int j = 0; j < VEC; ++j) W[j] = 0.0f;
  }
  if constexpr (HAS_EF) {
    float e[VEC];
    if (valid) {
      loadf<VEC>(ef + off, e);
    } else {
#pragma unroll
      for (int j = 0; j < VEC; ++j) e[j] = 0.0f;
    }
#pragma unroll
    for (int j = 0; j < VEC; ++j) v[j] = W[j] + e[j];
  } else {
#pragma unroll
    for (int j = 0; j < VEC; ++j) v[j] = W[j];
  }
  // W_hi
  uint32_t a = 0;
#pragma unroll
  for (int j = 0; j < VEC; ++j) a = umax(a, absbits(v[j]));
  a = seg_umax<G::L>(a);
  int e_hi = 0;
  float mul_hi, s_hi;
  if constexpr (F32S) {
    scale_from_amax(__uint_as_float(a), false, kE4M3Max, &mul_hi, &s_hi);
  } else {
    e_hi = block_exponent(__uint_as_float(a), kE4M3Max);
    mul_hi = exp2i(-e_hi);
    s_hi = exp2i(e_hi);
  }
  float c[VEC];
#pragma unroll
  for (int j = 0; j < VEC; ++j) c[j] = clampf(v[j] * mul_hi, kE4M3Max);
  uint32_t hc[VEC / 4];
  encode_words<VEC, TCFP_FP8_E4M3>(c, hc);
  float dh[VEC], r[VEC];
  uint32_t b = 0;
#pragma unroll
  for (int j = 0; j < VEC; ++j) {
    dh[j] = e4m3_to_f32(wbyte(hc, j)) * s_hi;
    r[j] = v[j] - dh[j];
    b = umax(b, absbits(r[j]));
  }
  // W_lo
  b = seg_umax<G::L>(b);
  const float amax_lo = __uint_as_float(b);
  const bool zero = !F32S && amax_lo < 1e-12f;
  int e_lo = 0;
  float mul_lo, inv_lo = 0.0f;
  if constexpr (F32S) {
    scale_from_amax(amax_lo, false, kE4M3Max, &mul_lo, &inv_lo);
  } else {
    e_lo = block_exponent(amax_lo, kE4M3Max);
    mul_lo = zero ? 1.0f : exp2i(-e_lo);
  }
#pragma unroll
  for (int j = 0; j < VEC; ++j) c[j] = clampf(r[j] * mul_lo, kE4M3Max);
  uint32_t lc[VEC / 4];
  if constexpr (SR) {
    // elements 8i .. 8i + 7 of the tensor (flat index) draw Philox counter
    // i; element 8i + j takes the 16-bit field j of the four output words
    static_assert(VEC % 8 == 0, "whole Philox calls per lane");
#pragma unroll
    for (int g8 = 0; g8 < VEC / 8; ++g8) {
      const uint64_t ctr = (uint64_t(off) >> 3) + uint64_t(g8);
      const u32x4 rr = philox4x32_10({uint32_t(ctr), uint32_t(ctr >> 32), off0, off1}, k0, k1);
      lc[2 * g8] = sr_block_hw4(c + 8 * g8, rr.x, rr.y);
      lc[2 * g8 + 1] = sr_block_hw4(c + 8 * g8 + 4, rr.z, rr.w);
    }
  } else {
    encode_words<VEC, TCFP_FP8_E4M3>(c, lc);
  }
  const int e_lo_store = zero ? -128 : e_lo;
  if (valid) {
    store_words<VEC>(hi + off, hc);
    store_words<VEC>(lo + off, lc);
    if (li == 0) {
      if constexpr (F32S) {
        static_cast<float*>(shi)[kb * n + row] = s_hi;
        static_cast<float*>(slo)[kb * n + row] = inv_lo;
      } else {
        static_cast<int8_t*>(shi)[kb * n + row] = int8_t(e_hi);
        static_cast<int8_t*>(slo)[kb * n + row] = int8_t(e_lo_store);
      }
    }
    if constexpr (HAS_EF && UPDATE) {
      const float s_lo = F32S ? inv_lo : exp2i(e_lo_store);
      float e[VEC];
#pragma unroll
      for (int j = 0; j < VEC; ++j) e[j] = (W[j] - dh[j]) - e4m3_to_f32(wbyte(lc, j)) * s_lo;
      storef<VEC>(ef + off, e);
    }
  }
}

template <int FMT, bool F32S>
__global__ __launch_bounds__(kThreads) void block_dequant_kernel(const uint8_t* __restrict__ q,
                                                                 const void* __restrict__ scales,
                                                                 int64_t m, int64_t k, int bs,
                                                                 float* __restrict__ out) {
  const int64_t n = m * k;
  const int64_t stride = int64_t(gridDim.x) * kThreads;
  for (int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x; i < n; i += stride) {
    const int64_t r = i / k, c = i - r * k;
    const int64_t si = (c / bs) * m + r;
    const float s = F32S ? static_cast<const float*>(scales)[si]
                         : exp2i(static_cast<const int8_t*>(scales)[si]);
    out[i] = fp8_to_f32<FMT>(q[i]) * s;
  }
}

// ===========================================================================
// Byte transpose through LDS (64x64 tiles)
// ===========================================================================
__global__ __launch_bounds__(kThreads) void transpose_u8_kernel(const uint8_t* __restrict__ src,
                                                                int64_t rows, int64_t cols,
                                                                uint8_t* __restrict__ dst) {
  __shared__ uint8_t tile[64][64 + 4];
  // one workgroup per 64 x 64 tile, tiles numbered row-major on a 1-D grid
  const int64_t tiles_c = (cols + 63) / 64;
  const int64_t r0 = int64_t(blockIdx.x) / tiles_c * 64, c0 = int64_t(blockIdx.x) % tiles_c * 64;
  const int t = threadIdx.x;
  const int lr = t >> 2, seg = t & 3;
  const int64_t r = r0 + lr;
#pragma unroll
  for (int b = 0; b < 16; ++b) {
    const int64_t c = c0 + seg * 16 + b;
    tile[lr][seg * 16 + b] = (r < rows && c < cols) ? src[r * cols + c] : 0;
  }
  __syncthreads();
  const int64_t c = c0 + lr;
  if (c < cols) {
#pragma unroll
    for (int b = 0; b < 16; ++b) {
      const int64_t rr = r0 + seg * 16 + b;
      if (rr < rows) dst[c * rows + rr] = tile[seg * 16 + b][lr];
    }
  }
}

// Launches transpose_u8_kernel over src [rows, cols] -> dst [cols, rows].
int launch_transpose_u8(const uint8_t* src, int64_t rows, int64_t cols, uint8_t* dst,
                        hipStream_t st) {
  const int64_t tiles = ((rows + 63) / 64) * ((cols + 63) / 64);
  if (!grid_x_fits(tiles, kThreads)) return TCFP_ERR_SHAPE;
  if (tiles > 0) transpose_u8_kernel<<<unsigned(tiles), kThreads, 0, st>>>(src, rows, cols, dst);
  return TCFP_OK;
}

// Re-blocking of a block dual-quantised weight W [rows, cols] (E4M3 codes,
// exponents [cols / bs, rows] along cols) along rows, in one pass: a
// workgroup takes a 128-row x 64-column tile of W_hi and W_lo, forms
// v = 2^e_hi W_hi + 2^e_lo W_lo in fp32 (an e_lo of -128 marks a zero
// residual block), holds v transposed in LDS, and dual-quantises each of the
// 64 transposed rows' 128 values in bs-wide blocks by the block_dualq_kernel
// rule (RNE, no EF): codes hi_t / lo_t [cols, rows], exponents [rows / bs,
// cols].  rows % bs == 0 (every block of a tile is whole), cols % 16 == 0.
template <int BS>
__global__ __launch_bounds__(kThreads) void requant_t_kernel(
    const uint8_t* __restrict__ hi, const uint8_t* __restrict__ lo,
    const int8_t* __restrict__ e_hi, const int8_t* __restrict__ e_lo, int64_t rows, int64_t cols,
    int bs_shift, uint8_t* __restrict__ hi_t, uint8_t* __restrict__ lo_t,
    int8_t* __restrict__ et_hi, int8_t* __restrict__ et_lo) {
  constexpr int TR = 128, TC = 64, VEC = 8, L = BS / VEC;
  __shared__ float tile[TC][TR + 1];
  const int64_t tiles_c = (cols + TC - 1) / TC;
  const int64_t r0 = int64_t(blockIdx.x) / tiles_c * TR, c0 = int64_t(blockIdx.x) % tiles_c * TC;
  const int t = threadIdx.x;
  // ---- v of 16 consecutive codes of one W row per thread and pass (they
  // share one block along cols, so one exponent per matrix)
  {
    const int lr = t >> 2, seg = t & 3;
    const int64_t cs = c0 + seg * 16;
#pragma unroll
    for (int p = 0; p < TR / 64; ++p) {
      const int tr = p * 64 + lr;
      const int64_t r = r0 + tr;
      float v[16];
      if (r < rows && cs < cols) {
        const int64_t kb = cs >> bs_shift;
        const float sh = exp2i(e_hi[kb * rows + r]);
        const uint4 qh = *reinterpret_cast<const uint4*>(hi + r * cols + cs);
        const uint32_t wh[4] = {qh.x, qh.y, qh.z, qh.w};
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = e4m3_to_f32(wbyte(wh, j)) * sh;
        const int el = lo ? int(e_lo[kb * rows + r]) : -128;
        if (el != -128) {
          const float sl = exp2i(el);
          const uint4 ql = *reinterpret_cast<const uint4*>(lo + r * cols + cs);
          const uint32_t wl[4] = {ql.x, ql.y, ql.z, ql.w};
#pragma unroll
          for (int j = 0; j < 16; ++j) v[j] = v[j] + e4m3_to_f32(wbyte(wl, j)) * sl;
        }
      } else {
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = 0.0f;
      }
#pragma unroll
      for (int j = 0; j < 16; ++j) tile[seg * 16 + j][tr] = v[j];
    }
  }
  __syncthreads();
  // ---- dual quantisation of the transposed rows: 16 lanes per row (VEC
  // values each), L lanes per bs-wide block
  const int part = t & 15;
#pragma unroll
  for (int p = 0; p < TC / 16; ++p) {
    const int oc = p * 16 + (t >> 4);
    const int64_t c = c0 + oc;
    const int64_t r = r0 + part * VEC;  // first value of this lane (a row of W)
    const bool valid = c < cols && r < rows;
    float v[VEC];
#pragma unroll
    for (int j = 0; j < VEC; ++j) v[j] = tile[oc][part * VEC + j];
    uint32_t a = 0;
#pragma unroll
    for (int j = 0; j < VEC; ++j) a = umax(a, absbits(v[j]));
    a = seg_umax<L>(a);
    const int eh = block_exponent(__uint_as_float(a), kE4M3Max);
    const float mul_hi = exp2i(-eh), s_hi = exp2i(eh);
    float cv[VEC];
#pragma unroll
    for (int j = 0; j < VEC; ++j) cv[j] = clampf(v[j] * mul_hi, kE4M3Max);
    uint32_t hc[VEC / 4];
    encode_words<VEC, TCFP_FP8_E4M3>(cv, hc);
    uint32_t b = 0;
    float res[VEC];
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      res[j] = v[j] - e4m3_to_f32(wbyte(hc, j)) * s_hi;
      b = umax(b, absbits(res[j]));
    }
    b = seg_umax<L>(b);
    const float amax_lo = __uint_as_float(b);
    const bool zero = amax_lo < 1e-12f;
    const int elo = block_exponent(amax_lo, kE4M3Max);
    const float mul_lo = zero ? 1.0f : exp2i(-elo);
#pragma unroll
    for (int j = 0; j < VEC; ++j) cv[j] = clampf(res[j] * mul_lo, kE4M3Max);
    uint32_t lc[VEC / 4];
    encode_words<VEC, TCFP_FP8_E4M3>(cv, lc);
    if (valid) {
      store_words<VEC>(hi_t + c * rows + r, hc);
      store_words<VEC>(lo_t + c * rows + r, lc);
      if (part % L == 0) {
        const int64_t kb = r >> bs_shift;
        et_hi[kb * cols + c] = int8_t(eh);
        et_lo[kb * cols + c] = int8_t(zero ? -128 : elo);
      }
    }
  }
}

// ===========================================================================
// Self tests
// ===========================================================================
template <int FMT>
__global__ __launch_bounds__(kThreads) void selftest_cvt_kernel(uint32_t lo, uint32_t hi,
                                                                unsigned long long* bad) {
  const uint64_t span = uint64_t(hi) - lo + 1;
  const uint64_t stride = uint64_t(gridDim.x) * kThreads;
  uint32_t cnt = 0;
  for (uint64_t i = uint64_t(blockIdx.x) * kThreads + threadIdx.x; i < span; i += stride) {
    const float x = __uint_as_float(lo + uint32_t(i));
    const uint32_t h = cvt4_fp8<FMT>(x, -x, 0.f, 0.f) & 0xFFFFu;
    const uint32_t s = f32_to_fp8<FMT>(x) | (f32_to_fp8<FMT>(-x) << 8);
    cnt += (h != s);
  }
  // workgroup 0 also decodes all 256 codes with both decoders
  if (blockIdx.x == 0) {
    const float a = fp8_to_f32<FMT>(threadIdx.x), b = sw_fp8_to_f32<FMT>(threadIdx.x);
    cnt += !((a != a && b != b) || __float_as_uint(a) == __float_as_uint(b));
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) cnt += __shfl_xor(cnt, o, 64);
  if ((threadIdx.x & 63) == 0 && cnt) atomicAdd(bad, (unsigned long long)cnt);
}

// sr_block (software converts) vs sr_block_hw and the packed sr_block_hw4
// on every float32 whose bit pattern lies in [lo, hi] and its negation, at
// one draw: u is truncated to k * 2^-16, the form the kernels draw.
__global__ __launch_bounds__(kThreads) void selftest_sr_kernel(uint32_t lo, uint32_t hi, float u,
                                                               unsigned long long* bad) {
  const uint64_t span = uint64_t(hi) - lo + 1;
  const uint64_t stride = uint64_t(gridDim.x) * kThreads;
  const uint32_t k = uint32_t(fminf(fmaxf(u, 0.0f), 0.99999f) * 65536.0f);
  const float uk = float(k) * 1.52587890625e-05f;
  const uint32_t r = k | (k << 16);
  uint32_t cnt = 0;
  for (uint64_t i = uint64_t(blockIdx.x) * kThreads + threadIdx.x; i < span; i += stride) {
    const float x = __uint_as_float(lo + uint32_t(i));
    const uint32_t a = sr_block(x, uk), b = sr_block(-x, uk);
    cnt += (a != sr_block_hw(x, uk));
    cnt += (b != sr_block_hw(-x, uk));
    const float c4[4] = {x, -x, -x, x};
    cnt += (sr_block_hw4(c4, r, r) != (a | (b << 8) | (b << 16) | (a << 24)));
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) cnt += __shfl_xor(cnt, o, 64);
  if ((threadIdx.x & 63) == 0 && cnt) atomicAdd(bad, (unsigned long long)cnt);
}

__global__ __launch_bounds__(kThreads) void selftest_philox_kernel(uint32_t c0, uint32_t c1,
                                                                   uint32_t c2, uint32_t c3,
                                                                   uint32_t k0, uint32_t k1,
                                                                   int64_t n, uint32_t* out) {
  const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= n) return;
  u32x4 r = philox4x32_10({c0 + uint32_t(i), c1, c2, c3}, k0, k1);
  out[4 * i] = r.x; out[4 * i + 1] = r.y; out[4 * i + 2] = r.z; out[4 * i + 3] = r.w;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

// ===========================================================================
// C ABI
// ===========================================================================
extern "C" {

const char* tcfp_status_string(int status) {
  switch (status) {
    case TCFP_OK: return "ok";
    case TCFP_ERR_SHAPE: return "invalid shape, leading dimension or divisibility";
    case TCFP_ERR_DTYPE: return "unsupported dtype or fp8 format";
    case TCFP_ERR_ALIGN: return "pointer or leading dimension not 16-byte aligned";
    case TCFP_ERR_HIP: return "HIP runtime error";
    case TCFP_ERR_WORKSPACE: return "workspace missing";
    case TCFP_ERR_EXCLUSIVE: return "stochastic_lo and error feedback are mutually exclusive";
    case TCFP_ERR_DEVICE: return "stream is not on the current device";
    default: return "unknown status";
  }
}

size_t tcfp_workspace_bytes(void) { return sizeof(PartWs); }

}  // extern "C"

namespace {

// pre_g > 0: a producer kernel already wrote pre_g partial maxima of the
// values to quantise to the workspace (no amax pass here).
// gelu_in: x is fp32 h and the values quantised are gelu(h), recomputed in
// the quantising pass (cols % 8 == 0).
// col_sum: the column sums of the values quantised, summed per 128-row tile
// by the tiled pass into cs_ws [ceil(rows / 128), cols], then over the
// tiles in order (cols % 8 == 0).
int quantize_impl(const void* x, int x_dtype, int64_t rows, int64_t cols, int fp8_fmt,
                  const float* scale_in, uint8_t* q, uint8_t* q_t, float* scale_out,
                  float* inv_out, void* workspace, float* col_sum, float* cs_ws,
                  hipStream_t st, int pre_g = 0, bool gelu_in = false, float* act_out = nullptr,
                  float* dg_out = nullptr) {
  if (rows < 0 || cols < 0) return TCFP_ERR_SHAPE;
  if (x_dtype != TCFP_DTYPE_F32 && x_dtype != TCFP_DTYPE_BF16) return TCFP_ERR_DTYPE;
  if (fp8_fmt != TCFP_FP8_E4M3 && fp8_fmt != TCFP_FP8_E5M2) return TCFP_ERR_DTYPE;
  if (!aligned16(x) || !inv_out) return TCFP_ERR_ALIGN;
  if (!scale_in && !workspace) return TCFP_ERR_WORKSPACE;
  if ((col_sum || gelu_in) && cols % 8 != 0) return TCFP_ERR_SHAPE;
  if (col_sum && gelu_in) return TCFP_ERR_SHAPE;
  if (gelu_in && x_dtype != TCFP_DTYPE_F32) return TCFP_ERR_DTYPE;
  if (!gelu_in && (act_out || dg_out)) return TCFP_ERR_SHAPE;
  if ((act_out && !aligned16(act_out)) || (dg_out && !aligned16(dg_out))) return TCFP_ERR_ALIGN;
  const int64_t n = rows * cols;
  if (n >= 8 && (reinterpret_cast<uintptr_t>(q) & 7u) != 0) return TCFP_ERR_ALIGN;
  PartWs* ws = static_cast<PartWs*>(workspace);
  const bool bf = x_dtype == TCFP_DTYPE_BF16;
  uint32_t* part = ws ? ws->a : nullptr;
  int g = 0;
  if (pre_g > 0) {
    g = pre_g;
  } else if (!scale_in && gelu_in) {
    g = gelu_grid(n);
    gelu_amax_kernel<<<g, kGeluThreads, 0, st>>>(static_cast<const float*>(x), n, nullptr, part);
  } else if (!scale_in) {
    g = parts_for((n + 7) / 8);
    if (bf)
      amax_part_kernel<uint16_t, false, false><<<g, kThreads, 0, st>>>(
          static_cast<const uint16_t*>(x), nullptr, n, part, nullptr, nullptr);
    else
      amax_part_kernel<float, false, false><<<g, kThreads, 0, st>>>(
          static_cast<const float*>(x), nullptr, n, part, nullptr, nullptr);
  }
  const int bfr = bf ? 1 : 0;
  const int64_t row_tiles = (rows + kTile - 1) / kTile;
  const bool tiled = (q_t || col_sum || gelu_in) && n > 0 && cols % 8 == 0;
  // the codes may be left out only where the tiled pass writes the
  // transposed copy instead
  if (!q && n > 0 && !(tiled && q_t)) return TCFP_ERR_SHAPE;
  if (tiled) {
    const int64_t tiles = int64_t(row_tiles) * ((cols + kTile - 1) / kTile);
    if (!grid_x_fits(tiles, kThreads)) return TCFP_ERR_SHAPE;
#define TCFP_QT(T, F, GL, CS)                                                                   \
  quant_t_kernel<T, F, GL, CS><<<unsigned(tiles), kThreads, 0, st>>>(                          \
      static_cast<const T*>(x), rows, cols, part, g, bfr, scale_in, q, q_t, scale_out, inv_out, \
      cs_ws, act_out, dg_out)
#define TCFP_QT_F(T, GL, CS)                                             \
  do {                                                                   \
    if (fp8_fmt == TCFP_FP8_E5M2) TCFP_QT(T, TCFP_FP8_E5M2, GL, CS);     \
    else TCFP_QT(T, TCFP_FP8_E4M3, GL, CS);                              \
  } while (0)
    if (gelu_in) {
      TCFP_QT_F(float, true, false);  // (no entry point asks for column sums of gelu(h))
    } else if (bf) {
      if (col_sum) TCFP_QT_F(uint16_t, false, true); else TCFP_QT_F(uint16_t, false, false);
    } else {
      if (col_sum) TCFP_QT_F(float, false, true); else TCFP_QT_F(float, false, false);
    }
#undef TCFP_QT_F
#undef TCFP_QT
    if (col_sum) {
      const int64_t groups = (rows + kColGroup - 1) / kColGroup;
      if (groups > INT32_MAX) return TCFP_ERR_SHAPE;
      colsum_finalize_kernel<<<unsigned((cols + 31) / 32), kThreads, 0, st>>>(cs_ws, int(groups),
                                                                              cols, col_sum);
    }
    return launch_status();
  }
  if (col_sum && cols > 0) {
    // no rows: the column sums are zero
    colsum_finalize_kernel<<<unsigned((cols + 31) / 32), kThreads, 0, st>>>(cs_ws, 0, cols,
                                                                            col_sum);
  }
  // flat (also for empty tensors: one workgroup still publishes scale / inv)
  const int gq = grid_for((n + 15) / 16, 8);
#define TCFP_QF(T, F)                                                                        \
  quant_flat_kernel<T, F><<<gq, kThreads, 0, st>>>(static_cast<const T*>(x), n, part, g, bfr, \
                                                    scale_in, q, scale_out, inv_out)
  if (bf) {
    if (fp8_fmt == TCFP_FP8_E5M2) TCFP_QF(uint16_t, TCFP_FP8_E5M2); else TCFP_QF(uint16_t, TCFP_FP8_E4M3);
  } else {
    if (fp8_fmt == TCFP_FP8_E5M2) TCFP_QF(float, TCFP_FP8_E5M2); else TCFP_QF(float, TCFP_FP8_E4M3);
  }
#undef TCFP_QF
  if (q_t && n > 0) {
    const int rc = launch_transpose_u8(q, rows, cols, q_t, st);
    if (rc != TCFP_OK) return rc;
  }
  return launch_status();
}

}  // namespace

namespace tcfp {

int max_parts() { return kMaxParts; }

namespace {
std::mutex g_premise_mu;
bool g_premise_launched[64] = {};

// Launches the premise check of the GELU amax rule on `st`, once per device
// and process.  Not while `st` is being captured (a graph would re-run it on
// every replay): until a later call launches it, the rule's users take the
// full pass.
void launch_gelu_premise_once(hipStream_t st) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return;
  std::lock_guard<std::mutex> lk(g_premise_mu);
  if (g_premise_launched[dev]) return;
  g_premise_launched[dev] = true;
  gelu_premise_check_kernel<<<kPremiseWgs, kThreads, 0, st>>>();
  gelu_premise_finalize_kernel<<<1, kThreads, 0, st>>>();
}
}  // namespace

int gelu_quantize_from_keys(const float* h, int64_t rows, int64_t cols, int fp8_fmt, float* act,
                            float* dgelu, uint8_t* q, uint8_t* q_t, float* inv_out,
                            void* workspace, const uint32_t* keys, int n_keys, void* stream) {
  if (rows < 0 || cols < 0 || cols % 8 != 0) return TCFP_ERR_SHAPE;
  if (!workspace) return TCFP_ERR_WORKSPACE;
  if (n_keys < 1 || n_keys > kMaxParts / 2 || !keys) return TCFP_ERR_SHAPE;
  const int64_t n = rows * cols;
  if (n == 0)
    return quantize_impl(h, TCFP_DTYPE_F32, rows, cols, fp8_fmt, nullptr, q, q_t, nullptr,
                         inv_out, workspace, nullptr, nullptr, static_cast<hipStream_t>(stream),
                         0, true, act, dgelu);
  hipStream_t st = static_cast<hipStream_t>(stream);
  launch_gelu_premise_once(st);
  PartWs* ws = static_cast<PartWs*>(workspace);
  // When the rule applies every workgroup only decides and writes its slot,
  // so the launch is sized for that: a quarter of the CUs (7.9 -> 4.5 us at
  // 32 Mi elements against a quarter of the usual grid).  The full pass it
  // falls back to (rare: a failed premise, NaN, -inf, all-negative h)
  // strides over h with that many workgroups.
  const int g = std::max(1, std::min(gelu_grid(n) / 4, num_cu() / 4));
  gelu_amax_rule_kernel<<<g, kGeluThreads, 0, st>>>(keys, n_keys, h, n, ws->gelu_rule, ws->a);
  return quantize_impl(h, TCFP_DTYPE_F32, rows, cols, fp8_fmt, nullptr, q, q_t, nullptr, inv_out,
                       workspace, nullptr, nullptr, st, g, true, act, dgelu);
}

int mul_quantize_colsum(const float* a, const float* b, int64_t rows, int64_t cols, int fp8_fmt,
                        float* out, uint8_t* q, uint8_t* q_t, float* inv_out, float* col_sum,
                        void* workspace, float* cs_ws, void* stream) {
  if (rows < 0 || cols < 0 || cols % 8 != 0) return TCFP_ERR_SHAPE;
  if (!workspace) return TCFP_ERR_WORKSPACE;
  if (!aligned16(a) || !aligned16(b) || !aligned16(out)) return TCFP_ERR_ALIGN;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t n = rows * cols;
  int g = 0;
  if (n > 0) {
    g = gelu_grid(n);
    mul_amax_kernel<<<g, kGeluThreads, 0, st>>>(a, b, n, out, static_cast<PartWs*>(workspace)->a);
  }
  return quantize_impl(out, TCFP_DTYPE_F32, rows, cols, fp8_fmt, nullptr, q, q_t, nullptr,
                       inv_out, workspace, col_sum, cs_ws, st, g);
}

int colsum_finalize(const float* cs_ws, int64_t groups, int64_t cols, float* col_sum,
                    void* stream) {
  if (cols <= 0) return TCFP_OK;
  if (groups < 0 || groups > INT32_MAX) return TCFP_ERR_SHAPE;
  colsum_finalize_kernel<<<unsigned((cols + 31) / 32), kThreads, 0,
                           static_cast<hipStream_t>(stream)>>>(cs_ws, int(groups), cols, col_sum);
  return launch_status();
}

int quantize_with_parts(const void* x, int x_dtype, int64_t rows, int64_t cols, int fp8_fmt,
                        uint8_t* q, uint8_t* q_t, float* inv_out, void* workspace,
                        float* col_sum, float* cs_ws, void* stream, int pre_g, bool gelu_in) {
  if (pre_g < 1 || pre_g > kMaxParts || !workspace) return TCFP_ERR_WORKSPACE;
  return quantize_impl(x, x_dtype, rows, cols, fp8_fmt, nullptr, q, q_t, nullptr, inv_out,
                       workspace, col_sum, cs_ws, static_cast<hipStream_t>(stream), pre_g,
                       gelu_in);
}

}  // namespace tcfp

extern "C" {

int tcfp_quantize_per_tensor(const void* x, int x_dtype, int64_t rows, int64_t cols,
                             int fp8_fmt, const float* scale_in, uint8_t* q, uint8_t* q_t,
                             float* scale_out, float* inv_out, void* workspace,
                             void* stream) {
  return quantize_impl(x, x_dtype, rows, cols, fp8_fmt, scale_in, q, q_t, scale_out, inv_out,
                       workspace, nullptr, nullptr, static_cast<hipStream_t>(stream));
}

int tcfp_quantize_per_tensor_sr(const void* x, int x_dtype, int64_t rows, int64_t cols,
                                const float* scale_in, uint64_t seed, uint64_t offset,
                                uint8_t* q, float* scale_out, float* inv_out, void* workspace,
                                void* stream) {
  if (rows < 0 || cols < 0) return TCFP_ERR_SHAPE;
  if (x_dtype != TCFP_DTYPE_F32 && x_dtype != TCFP_DTYPE_BF16) return TCFP_ERR_DTYPE;
  if (!aligned16(x) || !inv_out) return TCFP_ERR_ALIGN;
  if (!scale_in && !workspace) return TCFP_ERR_WORKSPACE;
  const int64_t n = rows * cols;
  if (n >= 8 && (reinterpret_cast<uintptr_t>(q) & 7u) != 0) return TCFP_ERR_ALIGN;
  hipStream_t st = static_cast<hipStream_t>(stream);
  PartWs* ws = static_cast<PartWs*>(workspace);
  uint32_t* part = ws ? ws->a : nullptr;
  const bool bf = x_dtype == TCFP_DTYPE_BF16;
  int g = 0;
  if (!scale_in) {
    g = parts_for((n + 7) / 8);
    if (bf)
      amax_part_kernel<uint16_t, false, false><<<g, kThreads, 0, st>>>(
          static_cast<const uint16_t*>(x), nullptr, n, part, nullptr, nullptr);
    else
      amax_part_kernel<float, false, false><<<g, kThreads, 0, st>>>(
          static_cast<const float*>(x), nullptr, n, part, nullptr, nullptr);
  }
  const int gq = grid_for((n + 7) / 8, 8);
  const uint32_t k0 = uint32_t(seed), k1 = uint32_t(seed >> 32);
  const uint32_t o0 = uint32_t(offset), o1 = uint32_t(offset >> 32);
  if (bf)
    quant_sr_kernel<uint16_t><<<gq, kThreads, 0, st>>>(static_cast<const uint16_t*>(x), n, part,
                                                       g, 1, scale_in, q, scale_out, inv_out, k0,
                                                       k1, o0, o1);
  else
    quant_sr_kernel<float><<<gq, kThreads, 0, st>>>(static_cast<const float*>(x), n, part, g, 0,
                                                    scale_in, q, scale_out, inv_out, k0, k1, o0,
                                                    o1);
  return launch_status();
}

int tcfp_block_scales(const void* x, int x_dtype, int64_t rows, int64_t cols, int block,
                      float fp8_max, void* scales, void* stream) {
  if (rows < 0 || cols < 0 || block <= 0 || cols % block != 0) return TCFP_ERR_SHAPE;
  if (!(fp8_max > 0.0f)) return TCFP_ERR_SHAPE;
  if (x_dtype != TCFP_DTYPE_F32 && x_dtype != TCFP_DTYPE_BF16) return TCFP_ERR_DTYPE;
  const int64_t nblocks = rows * (cols / block);
  if (nblocks == 0) return TCFP_OK;
  if (!x || !scales) return TCFP_ERR_SHAPE;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int gb = grid_for(nblocks, 8);
  if (x_dtype == TCFP_DTYPE_BF16)
    block_scales_kernel<uint16_t><<<gb, kThreads, 0, st>>>(
        static_cast<const uint16_t*>(x), nblocks, block, fp8_max, static_cast<uint16_t*>(scales));
  else
    block_scales_kernel<float><<<gb, kThreads, 0, st>>>(
        static_cast<const float*>(x), nblocks, block, fp8_max, static_cast<float*>(scales));
  return launch_status();
}

int tcfp_gelu_amax_rule_status(int* checked, int* holds, float* bound) {
  GeluPremise p;
  // the header words only (done, violations, t_bits)
  if (hipMemcpyFromSymbol(&p, HIP_SYMBOL(g_gelu_premise), 4 * sizeof(uint32_t), 0,
                          hipMemcpyDeviceToHost) != hipSuccess)
    return TCFP_ERR_HIP;
  if (checked) *checked = p.done == 1u ? 1 : 0;
  if (holds) *holds = (p.done == 1u && p.violations == 0u) ? 1 : 0;
  if (bound) std::memcpy(bound, &p.t_bits, sizeof(float));
  return TCFP_OK;
}

size_t tcfp_colsum_workspace_bytes(int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0 || cols % 8 != 0) return 0;
  return size_t((rows + kColGroup - 1) / kColGroup) * size_t(cols) * sizeof(float);
}

int tcfp_quantize_per_tensor_colsum(const void* x, int x_dtype, int64_t rows, int64_t cols,
                                    int fp8_fmt, uint8_t* q, uint8_t* q_t, float* inv_out,
                                    float* col_sum, void* workspace, void* colsum_ws,
                                    size_t colsum_ws_bytes, void* stream) {
  if (rows < 0 || cols < 0 || cols % 8 != 0) return TCFP_ERR_SHAPE;
  if (!col_sum) return TCFP_ERR_SHAPE;
  if (!workspace) return TCFP_ERR_WORKSPACE;
  if (rows > 0 && cols > 0 &&
      (!colsum_ws || colsum_ws_bytes < tcfp_colsum_workspace_bytes(rows, cols) ||
       !aligned16(colsum_ws) || !aligned16(col_sum)))
    return !colsum_ws || colsum_ws_bytes < tcfp_colsum_workspace_bytes(rows, cols)
               ? TCFP_ERR_WORKSPACE
               : TCFP_ERR_ALIGN;
  return quantize_impl(x, x_dtype, rows, cols, fp8_fmt, nullptr, q, q_t, nullptr, inv_out,
                       workspace, col_sum, static_cast<float*>(colsum_ws),
                       static_cast<hipStream_t>(stream));
}

int tcfp_gelu_quantize_per_tensor(const float* h, int64_t rows, int64_t cols, int fp8_fmt,
                                  float* act, float* dgelu, uint8_t* q, uint8_t* q_t,
                                  float* inv_out, void* workspace, void* stream) {
  if (rows < 0 || cols < 0) return TCFP_ERR_SHAPE;
  if (fp8_fmt != TCFP_FP8_E4M3 && fp8_fmt != TCFP_FP8_E5M2) return TCFP_ERR_DTYPE;
  if (!workspace) return TCFP_ERR_WORKSPACE;
  if (!aligned16(h) || (act && !aligned16(act)) || (dgelu && !aligned16(dgelu)) || !inv_out)
    return TCFP_ERR_ALIGN;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (cols % 8 == 0) {
    // the amax pass, then the quantising pass recomputes gelu(h) (and its
    // derivative factor) from h and writes what is asked for
    return quantize_impl(h, TCFP_DTYPE_F32, rows, cols, fp8_fmt, nullptr, q, q_t, nullptr,
                         inv_out, workspace, nullptr, nullptr, st, 0, true, act, dgelu);
  }
  // ragged rows: the amax pass writes gelu(h), which the flat pass quantises
  if (!act || dgelu) return TCFP_ERR_SHAPE;
  const int64_t n = rows * cols;
  const int g = gelu_grid(n);
  gelu_amax_kernel<<<g, kGeluThreads, 0, st>>>(h, n, act, static_cast<PartWs*>(workspace)->a);
  return quantize_impl(act, TCFP_DTYPE_F32, rows, cols, fp8_fmt, nullptr, q, q_t, nullptr,
                       inv_out, workspace, nullptr, nullptr, st, g);
}

int tcfp_gelu_backward_quantize_per_tensor_colsum(const float* dy, const float* h, int64_t rows,
                                                  int64_t cols, int fp8_fmt, float* grad,
                                                  uint8_t* q, uint8_t* q_t, float* inv_out,
                                                  float* col_sum, void* workspace,
                                                  void* colsum_ws, size_t colsum_ws_bytes,
                                                  void* stream) {
  if (rows < 0 || cols < 0 || cols % 8 != 0) return TCFP_ERR_SHAPE;
  if (fp8_fmt != TCFP_FP8_E4M3 && fp8_fmt != TCFP_FP8_E5M2) return TCFP_ERR_DTYPE;
  if (!workspace) return TCFP_ERR_WORKSPACE;
  if (!aligned16(dy) || !aligned16(h) || !aligned16(grad) || !inv_out) return TCFP_ERR_ALIGN;
  const int64_t n = rows * cols;
  if (col_sum && n > 0 &&
      (!colsum_ws || colsum_ws_bytes < tcfp_colsum_workspace_bytes(rows, cols)))
    return TCFP_ERR_WORKSPACE;
  if (col_sum && n > 0 && (!aligned16(colsum_ws) || !aligned16(col_sum))) return TCFP_ERR_ALIGN;
  hipStream_t st = static_cast<hipStream_t>(stream);
  int g = 0;
  if (n > 0) {
    g = gelu_grid(n);
    gelu_bwd_amax_kernel<<<g, kGeluThreads, 0, st>>>(dy, h, n, grad,
                                                     static_cast<PartWs*>(workspace)->a);
  }
  // an empty tensor has no partials: quantize_impl's own (empty) amax pass
  // publishes the clamped scale, as for any empty input
  return quantize_impl(grad, TCFP_DTYPE_F32, rows, cols, fp8_fmt, nullptr, q, q_t, nullptr,
                       inv_out, workspace, col_sum, static_cast<float*>(colsum_ws), st, g);
}

}  // extern "C"

namespace {

// Candidate pass of the per-tensor dual quantisation (set by
// tcfp_dual_quantize_set_candidates; on by default).
int g_cand_on = 1;

int dual_quantize_impl(const void* w, int w_dtype, int64_t n, int64_t k, float* ef,
                       int update_ef, int stochastic_lo, uint64_t seed, uint64_t offset,
                       uint8_t* w_hi, uint8_t* w_lo, float* inv_hi, float* inv_lo,
                       uint8_t* w_hi_t, uint8_t* w_lo_t, void* workspace, const Delayed& dl,
                       bool nf, float sigma, bool sr_hi, void* stream) {
  if (n < 0 || k < 0) return TCFP_ERR_SHAPE;
  if (w_dtype != TCFP_DTYPE_F32 && w_dtype != TCFP_DTYPE_BF16) return TCFP_ERR_DTYPE;
  if (!workspace) return TCFP_ERR_WORKSPACE;
  if (!aligned16(w) || !aligned16(w_hi) || !aligned16(w_lo) || (ef && !aligned16(ef)))
    return TCFP_ERR_ALIGN;
  hipStream_t st = static_cast<hipStream_t>(stream);
  PartWs* ws = static_cast<PartWs*>(workspace);
  const int64_t total = n * k;
  const int64_t nvec = (total + 7) / 8;
  const int ga = parts_for(nvec);
  const int gb = parts_for(nvec);
  const int gq = grid_for((nvec + 1) / 2, 8);
  const bool bf = w_dtype == TCFP_DTYPE_BF16;
  const bool has_ef = ef != nullptr;
  const bool upd = has_ef && update_ef;
  const bool tiled = (w_hi_t || w_lo_t) && total > 0 && k % 8 == 0;
  const int64_t tiles = ((n + kTile - 1) / kTile) * ((k + kTile - 1) / kTile);
  if (tiled && !grid_x_fits(tiles, kThreads)) return TCFP_ERR_SHAPE;
  const uint32_t k0 = uint32_t(seed), k1 = uint32_t(seed >> 32);
  const uint32_t o0 = uint32_t(offset), o1 = uint32_t(offset >> 32);

  HiRule hr{};
  if (nf) {
    hr.s1 = ws->s1;
    hr.s2 = ws->s2;
    hr.n = total;
    hr.sigma = sigma;
    hr.sr = sr_hi ? 1 : 0;
  }

  // Delayed scaling without validation predicts the residual amax: pass 2
  // (W_hi codes + residual amax) is skipped and pass 3 writes W_hi too.
  const bool two_pass = dl.on && !dl.validate;
  // The amax rule on a large tensor: pass 1 also keeps the candidates for
  // the residual amax in W_lo's buffer (one region of `cap` floats per
  // workgroup; W_lo is written last), a pass over them finds the residual
  // amax, and the full residual pass exits at once when they decide it
  // (cand_decisive); pass 3 then writes W_hi.
  const bool cand = g_cand_on && !nf && !dl.on && total >= (int64_t(1) << 23);
  const int cap = cand ? int(std::min<int64_t>(total / ga / 4, INT32_MAX)) : 0;
  // the candidate pass runs one workgroup per region, the full residual
  // pass behind it one per CU (it only does work when the candidates do not
  // decide); pass 3 reads gc or gbx partials
  const int gc = cand ? ga : 0;
  const int gbx = cand ? num_cu() : gb;
  uint32_t* const cand_cnt = reinterpret_cast<uint32_t*>(ws->s2);
  uint32_t* const cand_b2 = reinterpret_cast<uint32_t*>(ws->s1);
  const uint32_t* pb2 = cand ? cand_b2 : nullptr;
  uint8_t* hi3 = (two_pass || cand) ? w_hi : nullptr;
  // the residual pass takes the W_hi target from the W_hi pass when it ran
  const float* tgt3 = two_pass ? nullptr : &ws->hi_tgt;
#define TCFP_LO(T, EF, UP, SR)                                                                  \
  do {                                                                                          \
    if (tiled)                                                                                  \
      dualq_lo_t_kernel<T, EF, UP, SR><<<unsigned(tiles), kThreads, 0, st>>>(                   \
          wp, ef, n, k, ws->a, ga, ws->b, gbx, w_lo, inv_lo, w_hi_t, w_lo_t, k0, k1, o0, o1,     \
          dl, inv_hi, hi3, hr, tgt3, pb2, gc);                                                  \
    else                                                                                        \
      dualq_lo_kernel<T, EF, UP, SR><<<gq, kThreads, 0, st>>>(                                  \
          wp, ef, total, ws->a, ga, ws->b, gbx, w_lo, inv_lo, k0, k1, o0, o1, dl, inv_hi, hi3,   \
          hr, tgt3, pb2, gc);                                                                   \
  } while (0)
#define TCFP_DQ(T, EF)                                                                          \
  do {                                                                                          \
    const T* wp = static_cast<const T*>(w);                                                     \
    if (nf)                                                                                     \
      amax_part_kernel<T, EF, true><<<ga, kThreads, 0, st>>>(wp, ef, total, ws->a, ws->s1,     \
                                                             ws->s2);                           \
    else if (cand)                                                                              \
      amax_cand_kernel<T, EF><<<ga, kThreads, 0, st>>>(                                         \
          wp, ef, total, ws->a, CandOut{reinterpret_cast<float*>(w_lo), cand_cnt, cap});        \
    else                                                                                        \
      amax_part_kernel<T, EF, false><<<ga, kThreads, 0, st>>>(wp, ef, total, ws->a, nullptr,   \
                                                              nullptr);                         \
    if (cand)                                                                                   \
      cand_resid_kernel<<<gc, kThreads, 0, st>>>(reinterpret_cast<const float*>(w_lo),         \
                                                 cand_cnt, cap, ws->a, ga, cand_b2, inv_hi,     \
                                                 &ws->hi_tgt);                                  \
    if (!two_pass)                                                                              \
      dualq_hi_kernel<T, EF><<<gbx, kThreads, 0, st>>>(wp, ef, total, ws->a, ga,               \
                                                       cand ? nullptr : w_hi, ws->b, inv_hi,   \
                                                       dl, hr, k0, k1, o0, o1, &ws->hi_tgt,    \
                                                       pb2, gc);                               \
    if (stochastic_lo) {                                                                        \
      if (upd) TCFP_LO(T, EF, EF, true); else TCFP_LO(T, EF, false, true);                      \
    } else {                                                                                    \
      if (upd) TCFP_LO(T, EF, EF, false); else TCFP_LO(T, EF, false, false);                    \
    }                                                                                           \
  } while (0)

  if (bf) {
    if (has_ef) TCFP_DQ(uint16_t, true); else TCFP_DQ(uint16_t, false);
  } else {
    if (has_ef) TCFP_DQ(float, true); else TCFP_DQ(float, false);
  }
#undef TCFP_DQ
#undef TCFP_LO
  if (!tiled && total > 0 && (w_hi_t || w_lo_t)) {
    if (w_hi_t && launch_transpose_u8(w_hi, n, k, w_hi_t, st) != TCFP_OK) return TCFP_ERR_SHAPE;
    if (w_lo_t && launch_transpose_u8(w_lo, n, k, w_lo_t, st) != TCFP_OK) return TCFP_ERR_SHAPE;
  }
  return launch_status();
}

}  // namespace

namespace {

// ---- batched per-tensor quantisation (tcfp_quantize_batch) ----------------
// Each job keeps its own reduction workspace; a launch's workgroups are split
// among the jobs (job j owns [off[j], off[j + 1])) and each runs the
// single-tensor pass's body on its share.  In the amax and W_hi passes every
// job's share starts at a multiple of 8 workgroups, so a vector is handled
// on the same XCD (workgroup b runs on XCD b % 8) in both passes, as in the
// single-tensor launches.
constexpr int kMaxBatchJobs = 4;
struct BatchJob {
  const void* x;
  float* ef;
  int64_t rows, cols;
  int bf16, dual, has_ef, update, fmt;
  uint8_t* q;
  uint8_t* q_t;
  float* inv;
  uint8_t* q_lo;
  uint8_t* q_lo_t;
  float* inv_lo;
  PartWs* ws;
  int g1, g2;  // workgroups of the amax and W_hi passes
};
struct BatchArgs {
  BatchJob j[kMaxBatchJobs];
  int nj;
  int off[3][kMaxBatchJobs + 1];  // per pass: each job's first workgroup; [nj] = grid
};

// the job that workgroup blockIdx.x of pass p serves, and its index there
TCFP_DEV int batch_job(const BatchArgs& a, int p, int* bid) {
  int j = 0;
  while (j + 1 < a.nj && int(blockIdx.x) >= a.off[p][j + 1]) ++j;
  *bid = int(blockIdx.x) - a.off[p][j];
  return j;
}

__global__ __launch_bounds__(kThreads) void batch_amax_kernel(BatchArgs a) {
  __shared__ uint32_t red[kThreads / 64];
  __shared__ double rd[2 * (kThreads / 64)];
  int bid;
  const int j = batch_job(a, 0, &bid);
  const BatchJob& b = a.j[j];
  if (bid >= b.g1) return;  // (the padding up to a multiple of 8)
  const int64_t n = b.rows * b.cols;
  if (b.bf16) {
    const uint16_t* x = static_cast<const uint16_t*>(b.x);
    if (b.has_ef) amax_part_body<uint16_t, true, false>(x, b.ef, n, b.ws->a, nullptr, nullptr, bid, b.g1, red, rd);
    else amax_part_body<uint16_t, false, false>(x, nullptr, n, b.ws->a, nullptr, nullptr, bid, b.g1, red, rd);
  } else {
    const float* x = static_cast<const float*>(b.x);
    if (b.has_ef) amax_part_body<float, true, false>(x, b.ef, n, b.ws->a, nullptr, nullptr, bid, b.g1, red, rd);
    else amax_part_body<float, false, false>(x, nullptr, n, b.ws->a, nullptr, nullptr, bid, b.g1, red, rd);
  }
}

__global__ __launch_bounds__(kThreads) void batch_hi_kernel(BatchArgs a) {
  __shared__ uint32_t red[kThreads / 64];
  __shared__ uint32_t red2[kThreads / 64];
  __shared__ double rd[2 * (kThreads / 64)];
  int bid;
  const BatchJob& b = a.j[batch_job(a, 1, &bid)];
  if (bid >= b.g2) return;
  const int64_t n = b.rows * b.cols;
  const Delayed off{};
  const HiRule hr{};
#define TCFP_BHI(T, EF)                                                                        \
  dualq_hi_body<T, EF>(static_cast<const T*>(b.x), EF ? b.ef : nullptr, n, b.ws->a, b.g1, b.q, \
                       b.ws->b, b.inv, off, hr, 0, 0, 0, 0, &b.ws->hi_tgt, nullptr, 0, bid,   \
                       b.g2, red, red2, rd)
  if (b.bf16) {
    if (b.has_ef) TCFP_BHI(uint16_t, true); else TCFP_BHI(uint16_t, false);
  } else {
    if (b.has_ef) TCFP_BHI(float, true); else TCFP_BHI(float, false);
  }
#undef TCFP_BHI
}

__global__ __launch_bounds__(kThreads) void batch_final_kernel(BatchArgs a) {
  __shared__ uint32_t red[kThreads / 64];
  __shared__ uint32_t red2[kThreads / 64];
  __shared__ double rd[2 * (kThreads / 64)];
  __shared__ uint32_t tile_h[kTile * kTilePitch];
  __shared__ uint32_t tile_l[kTile * kTilePitch];
  int bid;
  const int j = batch_job(a, 2, &bid);
  const BatchJob& b = a.j[j];
  const int nbk = a.off[2][j + 1] - a.off[2][j];
  if (b.dual) {
    const Delayed off{};
    const HiRule hr{};
#define TCFP_BLO(T, EF, UP)                                                                    \
  dualq_lo_t_body<T, EF, UP, false>(static_cast<const T*>(b.x), EF ? b.ef : nullptr, b.rows,    \
                                    b.cols, b.ws->a, b.g1, b.ws->b, b.g2, b.q_lo, b.inv_lo,     \
                                    b.q_t, b.q_lo_t, 0, 0, 0, 0, off, nullptr, nullptr, hr,     \
                                    &b.ws->hi_tgt, nullptr, 0, bid, nbk, red, red2, rd, tile_h, \
                                    tile_l)
    if (b.bf16) {
      if (!b.has_ef) TCFP_BLO(uint16_t, false, false);
      else if (b.update) TCFP_BLO(uint16_t, true, true);
      else TCFP_BLO(uint16_t, true, false);
    } else {
      if (!b.has_ef) TCFP_BLO(float, false, false);
      else if (b.update) TCFP_BLO(float, true, true);
      else TCFP_BLO(float, true, false);
    }
#undef TCFP_BLO
  } else {
    float* const cs = reinterpret_cast<float*>(tile_l);  // (no column sums: unused)
#define TCFP_BQ(T, F)                                                                          \
  quant_t_body<T, F, false, false>(static_cast<const T*>(b.x), b.rows, b.cols, b.ws->a, b.g1,  \
                                   b.bf16, nullptr, b.q, b.q_t, nullptr, b.inv, nullptr,       \
                                   nullptr, nullptr, bid, nbk, red, tile_h, cs)
    if (b.bf16) {
      if (b.fmt == TCFP_FP8_E5M2) TCFP_BQ(uint16_t, TCFP_FP8_E5M2);
      else TCFP_BQ(uint16_t, TCFP_FP8_E4M3);
    } else {
      if (b.fmt == TCFP_FP8_E5M2) TCFP_BQ(float, TCFP_FP8_E5M2);
      else TCFP_BQ(float, TCFP_FP8_E4M3);
    }
#undef TCFP_BQ
  }
}

size_t batch_ws_bytes(int count) {
  return count > 0 ? size_t(count) * ((sizeof(PartWs) + 255) & ~size_t(255)) : 0;
}

}  // namespace

extern "C" {

size_t tcfp_quantize_batch_workspace_bytes(int count) {
  return count < 1 || count > kMaxBatchJobs ? 0 : batch_ws_bytes(count);
}

int tcfp_quantize_batch(int count, const tcfp_quant_job* jobs, void* workspace,
                        size_t workspace_bytes, void* stream) {
  if (count < 1 || count > kMaxBatchJobs || !jobs) return TCFP_ERR_SHAPE;
  if (!workspace || workspace_bytes < batch_ws_bytes(count)) return TCFP_ERR_WORKSPACE;
  if (!aligned16(workspace)) return TCFP_ERR_ALIGN;
  BatchArgs a{};
  a.nj = count;
  int o[3] = {0, 0, 0};
  for (int j = 0; j < count; ++j) {
    const tcfp_quant_job& s = jobs[j];
    BatchJob& b = a.j[j];
    if (s.kind != TCFP_JOB_DUAL && s.kind != TCFP_JOB_ACT) return TCFP_ERR_SHAPE;
    if (s.rows <= 0 || s.cols <= 0 || s.cols % 8 != 0) return TCFP_ERR_SHAPE;
    if (s.x_dtype != TCFP_DTYPE_F32 && s.x_dtype != TCFP_DTYPE_BF16) return TCFP_ERR_DTYPE;
    if (!s.x || !s.inv || !aligned16(s.x) || (s.ef && !aligned16(s.ef))) return TCFP_ERR_ALIGN;
    const bool dual = s.kind == TCFP_JOB_DUAL;
    if (dual) {
      if (!s.q || !s.q_lo || !s.inv_lo || !aligned16(s.q) || !aligned16(s.q_lo))
        return TCFP_ERR_ALIGN;
    } else {
      if (s.fp8_fmt != TCFP_FP8_E4M3 && s.fp8_fmt != TCFP_FP8_E5M2) return TCFP_ERR_DTYPE;
      if (!s.q && !s.q_t) return TCFP_ERR_SHAPE;
      if (s.q && (reinterpret_cast<uintptr_t>(s.q) & 7u) != 0) return TCFP_ERR_ALIGN;
    }
    const int64_t n = s.rows * s.cols;
    const int64_t tiles = ((s.rows + kTile - 1) / kTile) * ((s.cols + kTile - 1) / kTile);
    b.x = s.x;
    b.ef = dual ? s.ef : nullptr;
    b.rows = s.rows;
    b.cols = s.cols;
    b.bf16 = s.x_dtype == TCFP_DTYPE_BF16 ? 1 : 0;
    b.dual = dual ? 1 : 0;
    b.has_ef = b.ef ? 1 : 0;
    b.update = (b.ef && s.update_ef) ? 1 : 0;
    b.fmt = s.fp8_fmt;
    b.q = s.q;
    b.q_t = s.q_t;
    b.inv = s.inv;
    b.q_lo = dual ? s.q_lo : nullptr;
    b.q_lo_t = dual ? s.q_lo_t : nullptr;
    b.inv_lo = dual ? s.inv_lo : nullptr;
    b.ws = reinterpret_cast<PartWs*>(static_cast<uint8_t*>(workspace) +
                                     size_t(j) * ((sizeof(PartWs) + 255) & ~size_t(255)));
    b.g1 = parts_for((n + 7) / 8);
    b.g2 = dual ? parts_for((n + 7) / 8) : 0;
    a.off[0][j] = o[0];
    a.off[1][j] = o[1];
    a.off[2][j] = o[2];
    o[0] += (b.g1 + 7) / 8 * 8;
    o[1] += (b.g2 + 7) / 8 * 8;
    if (tiles > INT32_MAX - o[2]) return TCFP_ERR_SHAPE;
    o[2] += int(tiles);
  }
  for (int p = 0; p < 3; ++p) a.off[p][count] = o[p];
  hipStream_t st = static_cast<hipStream_t>(stream);
  batch_amax_kernel<<<unsigned(o[0]), kThreads, 0, st>>>(a);
  if (o[1] > 0) batch_hi_kernel<<<unsigned(o[1]), kThreads, 0, st>>>(a);
  batch_final_kernel<<<unsigned(o[2]), kThreads, 0, st>>>(a);
  return launch_status();
}

}  // extern "C"

extern "C" {

int tcfp_dual_quantize_set_candidates(int on) {
  if (on != 0 && on != 1) return TCFP_ERR_SHAPE;
  g_cand_on = on;
  return TCFP_OK;
}

int tcfp_dual_quantize_per_tensor(const void* w, int w_dtype, int64_t n, int64_t k,
                                  float* ef, int update_ef, int stochastic_lo,
                                  uint64_t seed, uint64_t offset, uint8_t* w_hi,
                                  uint8_t* w_lo, float* inv_hi, float* inv_lo,
                                  uint8_t* w_hi_t, uint8_t* w_lo_t, void* workspace,
                                  void* stream) {
  const Delayed off{};
  return dual_quantize_impl(w, w_dtype, n, k, ef, update_ef, stochastic_lo, seed, offset, w_hi,
                            w_lo, inv_hi, inv_lo, w_hi_t, w_lo_t, workspace, off, false, 0.0f,
                            false, stream);
}

}  // extern "C"

namespace {

// ---- scratch of the no-allocation entry point ----------------------------
// tcfp_dual_quantize_per_tensor_noalloc keeps its reduction partials in this
// file-scope device array instead of a caller workspace: one copy per GPU,
// held until the process ends.  On the host `scratch` names a host-side
// stand-in, not device memory, so host code never passes it to a kernel: the
// device address comes from hipGetSymbolAddress, looked up once per device
// (with that device current, on the first call there) and kept in
// g_scratch_ptr.  Every call on a GPU shares that GPU's array.  The
// reduction partials need no initialisation (each launch writes the slots it
// reads before reading them), so nothing is cleared between calls.
constexpr size_t kScratchBytes = 49408;  // the per-tensor reductions' PartWs
static_assert(sizeof(PartWs) <= kScratchBytes, "scratch must hold the reduction workspace");
static __device__ __align__(256) uint8_t scratch[kScratchBytes];
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of this GPU's scratch; the stream must belong to the
// current device.
int scratch_for(hipStream_t st, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) return TCFP_ERR_HIP;
  if (dev < 0 || dev >= kMaxDevices) return TCFP_ERR_DEVICE;
  if (st != nullptr) {
    hipDevice_t sd = -1;
    if (hipStreamGetDevice(st, &sd) != hipSuccess) return TCFP_ERR_HIP;
    if (sd != dev) return TCFP_ERR_DEVICE;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || ptr == nullptr)
      return TCFP_ERR_HIP;
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return TCFP_OK;
}

}  // namespace

extern "C" {

int tcfp_dual_quantize_per_tensor_noalloc(const void* w, int w_dtype, int64_t n, int64_t k,
                                          float* ef, int update_ef, int stochastic_lo,
                                          uint64_t seed, uint64_t offset, uint8_t* w_hi,
                                          uint8_t* w_lo, float* inv_hi, float* inv_lo,
                                          uint8_t* w_hi_t, uint8_t* w_lo_t, void* stream) {
  if (tcfp_workspace_bytes() > kScratchBytes) return TCFP_ERR_WORKSPACE;
  void* ws = nullptr;
  const int rc = scratch_for(static_cast<hipStream_t>(stream), &ws);
  if (rc != TCFP_OK) return rc;
  const Delayed off{};
  return dual_quantize_impl(w, w_dtype, n, k, ef, update_ef, stochastic_lo, seed, offset, w_hi,
                            w_lo, inv_hi, inv_lo, w_hi_t, w_lo_t, ws, off, false, 0.0f, false,
                            stream);
}

int tcfp_dual_quantize_per_tensor_delayed(const void* w, int w_dtype, int64_t n, int64_t k,
                                          float* ef, int update_ef, const float* amax_prev,
                                          const float* ratio_prev, float ema_decay,
                                          float one_minus_decay, int validate, float* amax_out,
                                          float* ratio_out, uint8_t* w_hi, uint8_t* w_lo,
                                          float* inv_hi, float* inv_lo, uint8_t* w_hi_t,
                                          uint8_t* w_lo_t, void* workspace, void* stream) {
  if (!amax_out || (validate && !ratio_out) || !inv_hi || !inv_lo) return TCFP_ERR_SHAPE;
  if (n * k == 0) return TCFP_ERR_SHAPE;  // the reference's amax of an empty tensor raises
  Delayed dl{};
  dl.amax_prev = amax_prev;
  dl.ratio_prev = ratio_prev;
  dl.amax_out = amax_out;
  dl.ratio_out = ratio_out;
  dl.a = ema_decay;
  dl.b = one_minus_decay;
  dl.on = 1;
  dl.validate = validate ? 1 : 0;
  return dual_quantize_impl(w, w_dtype, n, k, ef, update_ef, 0, 0, 0, w_hi, w_lo, inv_hi, inv_lo,
                            w_hi_t, w_lo_t, workspace, dl, false, 0.0f, false, stream);
}

int tcfp_dual_quantize_per_tensor_nf(const void* w, int w_dtype, int64_t n, int64_t k, float* ef,
                                     int update_ef, float sigma_factor, int stochastic_hi,
                                     int stochastic_lo, uint64_t seed, uint64_t offset,
                                     const float* amax_prev, const float* ratio_prev,
                                     float ema_decay, float one_minus_decay, int validate,
                                     float* amax_out, float* ratio_out, uint8_t* w_hi,
                                     uint8_t* w_lo, float* inv_hi, float* inv_lo,
                                     uint8_t* w_hi_t, uint8_t* w_lo_t, void* workspace,
                                     void* stream) {
  if (!inv_hi || !inv_lo) return TCFP_ERR_SHAPE;
  // the reference's residual amax of an empty tensor raises
  if (n * k == 0) return TCFP_ERR_SHAPE;
  Delayed dl{};
  if (amax_out) {
    if (validate && !ratio_out) return TCFP_ERR_SHAPE;
    dl.amax_prev = amax_prev;
    dl.ratio_prev = ratio_prev;
    dl.amax_out = amax_out;
    dl.ratio_out = ratio_out;
    dl.a = ema_decay;
    dl.b = one_minus_decay;
    dl.on = 1;
    dl.validate = validate ? 1 : 0;
  }
  return dual_quantize_impl(w, w_dtype, n, k, ef, update_ef, stochastic_lo, seed, offset, w_hi,
                            w_lo, inv_hi, inv_lo, w_hi_t, w_lo_t, workspace, dl, true,
                            sigma_factor, stochastic_hi != 0, stream);
}

}  // extern "C"

namespace {

template <bool F32S>
int block_quantize_impl(const void* x, int x_dtype, int64_t m, int64_t k, int block, int fp8_fmt,
                        uint8_t* q, void* scales, hipStream_t st) {
  if (m < 0 || k < 0) return TCFP_ERR_SHAPE;
  if (block != 32 && block != 64 && block != 128) return TCFP_ERR_SHAPE;
  if (k % block != 0) return TCFP_ERR_SHAPE;
  if (x_dtype != TCFP_DTYPE_F32 && x_dtype != TCFP_DTYPE_BF16) return TCFP_ERR_DTYPE;
  if (fp8_fmt != TCFP_FP8_E4M3 && fp8_fmt != TCFP_FP8_E5M2) return TCFP_ERR_DTYPE;
  if (!aligned16(x) || !aligned16(q)) return TCFP_ERR_ALIGN;
  if (m == 0 || k == 0) return TCFP_OK;
  if (m > INT32_MAX) return TCFP_ERR_SHAPE;
  const unsigned kbs = unsigned(k / block);
  // (grid y holds at most 65535 K-blocks)
  const bool kfast = m * k * (x_dtype == TCFP_DTYPE_F32 ? 4 : 2) >= kKFastBytes || kbs > 65535u;
#define TCFP_BQ(T, F, B)                                                                    \
  do {                                                                                      \
    const int64_t rgs = (m + Seg<T, B>::ROWS - 1) / Seg<T, B>::ROWS;                        \
    if (!grid_x_fits(kfast ? rgs * kbs : rgs, kThreads)) return TCFP_ERR_SHAPE;              \
    const dim3 grid = kfast ? dim3(unsigned(rgs * kbs)) : dim3(unsigned(rgs), kbs);         \
    block_quant_kernel<T, F, B, F32S><<<grid, kThreads, 0, st>>>(static_cast<const T*>(x),  \
                                                                 m, k, q, scales, kfast);   \
  } while (0)
#define TCFP_BQ_B(T, F)                                 \
  do {                                                  \
    if (block == 32) TCFP_BQ(T, F, 32);                 \
    else if (block == 64) TCFP_BQ(T, F, 64);            \
    else TCFP_BQ(T, F, 128);                            \
  } while (0)
  if (x_dtype == TCFP_DTYPE_BF16) {
    if (fp8_fmt == TCFP_FP8_E5M2) TCFP_BQ_B(uint16_t, TCFP_FP8_E5M2); else TCFP_BQ_B(uint16_t, TCFP_FP8_E4M3);
  } else {
    if (fp8_fmt == TCFP_FP8_E5M2) TCFP_BQ_B(float, TCFP_FP8_E5M2); else TCFP_BQ_B(float, TCFP_FP8_E4M3);
  }
#undef TCFP_BQ_B
#undef TCFP_BQ
  return launch_status();
}

template <bool F32S>
int block_dual_quantize_impl(const void* w, int w_dtype, int64_t n, int64_t k, int block,
                             float* ef, int update_ef, int stochastic_lo, uint64_t seed,
                             uint64_t offset, uint8_t* w_hi, uint8_t* w_lo, void* s_hi,
                             void* s_lo, hipStream_t st) {
  if (n < 0 || k < 0) return TCFP_ERR_SHAPE;
  if (block != 32 && block != 64 && block != 128) return TCFP_ERR_SHAPE;
  if (k % block != 0) return TCFP_ERR_SHAPE;
  if (w_dtype != TCFP_DTYPE_F32 && w_dtype != TCFP_DTYPE_BF16) return TCFP_ERR_DTYPE;
  if (stochastic_lo && ef) return TCFP_ERR_EXCLUSIVE;
  if (!aligned16(w) || !aligned16(w_hi) || !aligned16(w_lo) || (ef && !aligned16(ef)))
    return TCFP_ERR_ALIGN;
  if (n == 0 || k == 0) return TCFP_OK;
  if (n > INT32_MAX) return TCFP_ERR_SHAPE;
  const unsigned kbs = unsigned(k / block);
  // (grid y holds at most 65535 K-blocks)
  const bool kfast = n * k * (w_dtype == TCFP_DTYPE_F32 ? 4 : 2) >= kKFastBytes || kbs > 65535u;
  const uint32_t k0 = uint32_t(seed), k1 = uint32_t(seed >> 32);
  const uint32_t o0 = uint32_t(offset), o1 = uint32_t(offset >> 32);
  const bool upd = ef && update_ef;
#define TCFP_BDQ(T, B, EF, UP, SR)                                                             \
  do {                                                                                         \
    using DS = DualSeg<T, B, SR>;                                                              \
    const int64_t rgs = (n + DS::ROWS - 1) / DS::ROWS;                                         \
    if (!grid_x_fits(kfast ? rgs * kbs : rgs, kThreads)) return TCFP_ERR_SHAPE;                 \
    const dim3 grid = kfast ? dim3(unsigned(rgs * kbs)) : dim3(unsigned(rgs), kbs);            \
    block_dualq_kernel<T, B, EF, UP, SR, F32S><<<grid, kThreads, 0, st>>>(                     \
        static_cast<const T*>(w), ef, n, k, w_hi, w_lo, s_hi, s_lo, k0, k1, o0, o1, kfast);    \
  } while (0)
#define TCFP_BDQ_MODE(T, B)                                     \
  do {                                                          \
    if (stochastic_lo) TCFP_BDQ(T, B, false, false, true);      \
    else if (ef && upd) TCFP_BDQ(T, B, true, true, false);      \
    else if (ef) TCFP_BDQ(T, B, true, false, false);            \
    else TCFP_BDQ(T, B, false, false, false);                   \
  } while (0)
#define TCFP_BDQ_B(T)                                 \
  do {                                                \
    if (block == 32) TCFP_BDQ_MODE(T, 32);            \
    else if (block == 64) TCFP_BDQ_MODE(T, 64);       \
    else TCFP_BDQ_MODE(T, 128);                       \
  } while (0)
  if (w_dtype == TCFP_DTYPE_BF16) TCFP_BDQ_B(uint16_t); else TCFP_BDQ_B(float);
#undef TCFP_BDQ_B
#undef TCFP_BDQ_MODE
#undef TCFP_BDQ
  return launch_status();
}

template <bool F32S>
int block_dequantize_impl(const uint8_t* q, int fp8_fmt, const void* scales, int64_t m,
                          int64_t k, int block, float* out, hipStream_t st) {
  if (m < 0 || k < 0 || block <= 0 || k % block != 0) return TCFP_ERR_SHAPE;
  if (fp8_fmt != TCFP_FP8_E4M3 && fp8_fmt != TCFP_FP8_E5M2) return TCFP_ERR_DTYPE;
  if (m == 0 || k == 0) return TCFP_OK;
  const int g = grid_for(m * k, 16);
  if (fp8_fmt == TCFP_FP8_E5M2)
    block_dequant_kernel<TCFP_FP8_E5M2, F32S><<<g, kThreads, 0, st>>>(q, scales, m, k, block, out);
  else
    block_dequant_kernel<TCFP_FP8_E4M3, F32S><<<g, kThreads, 0, st>>>(q, scales, m, k, block, out);
  return launch_status();
}

}  // namespace

extern "C" {

int tcfp_block_quantize(const void* x, int x_dtype, int64_t m, int64_t k, int block,
                        int fp8_fmt, uint8_t* q, int8_t* exps, void* stream) {
  return block_quantize_impl<false>(x, x_dtype, m, k, block, fp8_fmt, q, exps,
                                    static_cast<hipStream_t>(stream));
}

int tcfp_block_quantize_f32s(const void* x, int x_dtype, int64_t m, int64_t k, int block,
                             int fp8_fmt, uint8_t* q, float* inv_scales, void* stream) {
  return block_quantize_impl<true>(x, x_dtype, m, k, block, fp8_fmt, q, inv_scales,
                                   static_cast<hipStream_t>(stream));
}

int tcfp_block_dual_quantize(const void* w, int w_dtype, int64_t n, int64_t k, int block,
                             float* ef, int update_ef, int stochastic_lo, uint64_t seed,
                             uint64_t offset, uint8_t* w_hi, uint8_t* w_lo, int8_t* e_hi,
                             int8_t* e_lo, void* stream) {
  return block_dual_quantize_impl<false>(w, w_dtype, n, k, block, ef, update_ef, stochastic_lo,
                                         seed, offset, w_hi, w_lo, e_hi, e_lo,
                                         static_cast<hipStream_t>(stream));
}

int tcfp_block_dual_quantize_f32s(const void* w, int w_dtype, int64_t n, int64_t k, int block,
                                  float* ef, int update_ef, int stochastic_lo, uint64_t seed,
                                  uint64_t offset, uint8_t* w_hi, uint8_t* w_lo, float* inv_hi,
                                  float* inv_lo, void* stream) {
  return block_dual_quantize_impl<true>(w, w_dtype, n, k, block, ef, update_ef, stochastic_lo,
                                        seed, offset, w_hi, w_lo, inv_hi, inv_lo,
                                        static_cast<hipStream_t>(stream));
}

int tcfp_block_requant_t(const uint8_t* w_hi, const uint8_t* w_lo, const int8_t* e_hi,
                         const int8_t* e_lo, int64_t d_out, int64_t d_in, int block,
                         uint8_t* wt_hi, uint8_t* wt_lo, int8_t* et_hi, int8_t* et_lo,
                         void* stream) {
  if (d_out < 0 || d_in < 0) return TCFP_ERR_SHAPE;
  if (block != 32 && block != 64 && block != 128) return TCFP_ERR_SHAPE;
  if (d_out % block != 0 || d_in % block != 0) return TCFP_ERR_SHAPE;
  if (!w_hi || !e_hi || !wt_hi || !wt_lo || !et_hi || !et_lo) return TCFP_ERR_SHAPE;
  if ((w_lo == nullptr) != (e_lo == nullptr)) return TCFP_ERR_SHAPE;
  if (!aligned16(w_hi) || (w_lo && !aligned16(w_lo)) || !aligned16(wt_hi) || !aligned16(wt_lo))
    return TCFP_ERR_ALIGN;
  if (d_out == 0 || d_in == 0) return TCFP_OK;
  const int64_t tiles = ((d_out + 127) / 128) * ((d_in + 63) / 64);
  if (!grid_x_fits(tiles, kThreads)) return TCFP_ERR_SHAPE;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const unsigned g = unsigned(tiles);
  if (block == 32)
    requant_t_kernel<32><<<g, kThreads, 0, st>>>(w_hi, w_lo, e_hi, e_lo, d_out, d_in, 5, wt_hi,
                                                 wt_lo, et_hi, et_lo);
  else if (block == 64)
    requant_t_kernel<64><<<g, kThreads, 0, st>>>(w_hi, w_lo, e_hi, e_lo, d_out, d_in, 6, wt_hi,
                                                 wt_lo, et_hi, et_lo);
  else
    requant_t_kernel<128><<<g, kThreads, 0, st>>>(w_hi, w_lo, e_hi, e_lo, d_out, d_in, 7, wt_hi,
                                                  wt_lo, et_hi, et_lo);
  return launch_status();
}

int tcfp_block_dequantize(const uint8_t* q, int fp8_fmt, const int8_t* exps, int64_t m,
                          int64_t k, int block, float* out, void* stream) {
  return block_dequantize_impl<false>(q, fp8_fmt, exps, m, k, block, out,
                                      static_cast<hipStream_t>(stream));
}

int tcfp_block_dequantize_f32s(const uint8_t* q, int fp8_fmt, const float* inv_scales, int64_t m,
                               int64_t k, int block, float* out, void* stream) {
  return block_dequantize_impl<true>(q, fp8_fmt, inv_scales, m, k, block, out,
                                     static_cast<hipStream_t>(stream));
}

int tcfp_transpose_u8(const uint8_t* src, int64_t rows, int64_t cols, uint8_t* dst,
                      void* stream) {
  if (rows < 0 || cols < 0) return TCFP_ERR_SHAPE;
  if (rows == 0 || cols == 0) return TCFP_OK;
  const int rc = launch_transpose_u8(src, rows, cols, dst, static_cast<hipStream_t>(stream));
  return rc != TCFP_OK ? rc : launch_status();
}

int tcfp_selftest_fp8_cvt(uint32_t lo_bits, uint32_t hi_bits, int fp8_fmt,
                          unsigned long long* mismatches, void* stream) {
  if (hi_bits < lo_bits) return TCFP_ERR_SHAPE;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int g = num_cu() * 8;
  if (fp8_fmt == TCFP_FP8_E5M2)
    selftest_cvt_kernel<TCFP_FP8_E5M2><<<g, kThreads, 0, st>>>(lo_bits, hi_bits, mismatches);
  else if (fp8_fmt == TCFP_FP8_E4M3)
    selftest_cvt_kernel<TCFP_FP8_E4M3><<<g, kThreads, 0, st>>>(lo_bits, hi_bits, mismatches);
  else
    return TCFP_ERR_DTYPE;
  return launch_status();
}

int tcfp_selftest_sr_block(uint32_t lo_bits, uint32_t hi_bits, float u,
                           unsigned long long* mismatches, void* stream) {
  if (hi_bits < lo_bits || hi_bits > 0x43E00000u) return TCFP_ERR_SHAPE;
  const int g = num_cu() * 8;
  selftest_sr_kernel<<<g, kThreads, 0, static_cast<hipStream_t>(stream)>>>(lo_bits, hi_bits, u,
                                                                           mismatches);
  return launch_status();
}

int tcfp_selftest_philox(uint32_t ctr0, uint32_t ctr1, uint32_t ctr2, uint32_t ctr3,
                         uint32_t k0, uint32_t k1, int64_t n, uint32_t* out, void* stream) {
  if (n <= 0) return n == 0 ? TCFP_OK : TCFP_ERR_SHAPE;
  const int g = int((n + kThreads - 1) / kThreads);
  selftest_philox_kernel<<<g, kThreads, 0, static_cast<hipStream_t>(stream)>>>(
      ctr0, ctr1, ctr2, ctr3, k0, k1, n, out);
  return launch_status();
}

}  // extern "C"
