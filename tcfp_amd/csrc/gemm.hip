// FP8 GEMMs for the TCFP-12 path on gfx950 (CDNA4 MFMA).
//
// One kernel shape serves every GEMM of the path because every operand is
// produced K-contiguous ("NT": A [M,K], B [N,K], both row-major):
//   forward   out  = X W_hi^T s_x s_hi + X W_lo^T s_x s_lo       (dual)
//   dgrad     dX   = G W_hi s_g s_hi + G W_lo s_g s_lo            (dual, B = W^T copies)
//   wgrad     dW   = G^T X s_g s_x                                (single, A = G^T, B = X^T)
// The quantisation kernels emit the transposed copies, so no GEMM needs a
// transposing operand path.
//
// Tiling: a 256-thread workgroup (4 wave64s, one per SIMD) owns a 256 x 128
// output tile.  Per K step the A tile (256 x BK) is staged once in LDS and
// shared by the two B tiles (W_hi and W_lo, 128 x BK each) -- the dual GEMM
// is a single GEMM over [W_hi; W_lo] whose two accumulator halves meet in
// the epilogue.  Each wave computes 128 x 64 of both halves with
// v_mfma_scale_f32_32x32x64_f8f6f4 (neutral E8M0 scales), i.e. 4 x 2 x 2
// 32x32 accumulator tiles (256 fp32 per lane).  In single-GEMM mode the two
// B slots hold adjacent 128-column halves of one 256-wide tile.
//
// LDS rows are 16-byte-chunk XOR-swizzled so that both the 16-byte global
// -> LDS stores and the 32-byte-per-lane MFMA operand reads are free of
// bank conflicts.  Two LDS stages with register prefetch overlap the next
// tile's global loads with the current tile's MFMAs; one barrier per step.
//
// Workgroup -> tile mapping is XCD-aware: the dispatcher places workgroup b
// on XCD b % 8, so workgroups are renumbered to give each XCD a contiguous
// run of tiles, grouped 8 tile-rows deep, which keeps an XCD's A and B
// panels resident in its own L2.
#include "common.h"

using namespace tcfp;

namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kNT = 256;
constexpr int kBM = 256;
constexpr int kBN = 128;

template <int BK>
struct Lds {
  static constexpr int CPR = BK / 16;    // 16-byte chunks per row
  static constexpr int RPW = 256 / BK;   // rows per 256-byte bank window
  static constexpr int A = kBM * BK;
  static constexpr int B = kBN * BK;
  static constexpr int STAGE = A + 2 * B;
  // byte offset of chunk `ch` of row `r`
  static TCFP_DEV int off(int r, int ch) { return r * BK + (((ch ^ (r / RPW)) & (CPR - 1)) << 4); }
};

TCFP_DEV uint4 lds_read16(const uint8_t* base, int off) {
  return *reinterpret_cast<const uint4*>(base + off);
}

TCFP_DEV v8i make_frag(uint4 lo, uint4 hi) {
  v8i f;
  f[0] = int(lo.x); f[1] = int(lo.y); f[2] = int(lo.z); f[3] = int(lo.w);
  f[4] = int(hi.x); f[5] = int(hi.y); f[6] = int(hi.z); f[7] = int(hi.w);
  return f;
}

template <typename OutT>
TCFP_DEV void store_out(OutT* p, float v);
template <>
TCFP_DEV void store_out<float>(float* p, float v) { *p = v; }
template <>
TCFP_DEV void store_out<uint16_t>(uint16_t* p, float v) { *p = f32_to_bf16_rne(v); }

// AF/BF: fp8 format codes of A and B (0 = E4M3, 1 = E5M2), matching the
// MFMA cbsz/blgp format selectors.  SPLIT = single-GEMM mode.
template <int AF, int BF, bool SPLIT, int BK, typename OutT>
__global__ __launch_bounds__(kNT, 1) void gemm_nt_kernel(
    const uint8_t* __restrict__ A, const uint8_t* __restrict__ B0, const uint8_t* __restrict__ B1,
    int M, int N, int K, int64_t lda, int64_t ldb, const float* __restrict__ s_a,
    const float* __restrict__ s_0, const float* __restrict__ s_1, const float* __restrict__ bias,
    OutT* __restrict__ out, int64_t ldo, int tiles_m, int tiles_n) {
  using L = Lds<BK>;
  extern __shared__ __align__(16) uint8_t smem[];

  // ---- tile mapping (XCD-aware, grouped) ----
  const int T = tiles_m * tiles_n;
  int l = blockIdx.x;
  if ((T & 7) == 0) l = (l & 7) * (T >> 3) + (l >> 3);
  constexpr int G = 8;
  const int per_group = G * tiles_n;
  const int first_m = (l / per_group) * G;
  const int gm = min(tiles_m - first_m, G);
  const int tm = first_m + (l % per_group) % gm;
  const int tn = (l % per_group) / gm;
  const int m0 = tm * kBM;
  const int n0 = SPLIT ? tn * (2 * kBN) : tn * kBN;
  const int n1 = SPLIT ? n0 + kBN : n0;  // row base of the second B slot

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int lr = lane & 31, lg = lane >> 5;

  // ---- global -> register prefetch mapping ----
  constexpr int A_CH = kBM * L::CPR / kNT;  // 16-byte chunks per thread for A
  constexpr int B_CH = kBN * L::CPR / kNT;  // ... for each B slot
  uint4 pa[A_CH], pb0[B_CH], pb1[B_CH];

  auto gload = [&](int kt) {
    const int kbase = kt * BK;
#pragma unroll
    for (int i = 0; i < A_CH; ++i) {
      const int c = tid + i * kNT;
      const int r = c / L::CPR, ch = c % L::CPR;
      const int gr = m0 + r, gk = kbase + ch * 16;
      pa[i] = (gr < M && gk < K) ? *reinterpret_cast<const uint4*>(A + int64_t(gr) * lda + gk)
                                 : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < B_CH; ++i) {
      const int c = tid + i * kNT;
      const int r = c / L::CPR, ch = c % L::CPR;
      const int gk = kbase + ch * 16;
      const int g0 = n0 + r, g1 = n1 + r;
      pb0[i] = (g0 < N && gk < K) ? *reinterpret_cast<const uint4*>(B0 + int64_t(g0) * ldb + gk)
                                  : make_uint4(0, 0, 0, 0);
      pb1[i] = (g1 < N && gk < K) ? *reinterpret_cast<const uint4*>(B1 + int64_t(g1) * ldb + gk)
                                  : make_uint4(0, 0, 0, 0);
    }
  };
  auto lstore = [&](int stage) {
    uint8_t* base = smem + stage * L::STAGE;
#pragma unroll
    for (int i = 0; i < A_CH; ++i) {
      const int c = tid + i * kNT;
      *reinterpret_cast<uint4*>(base + L::off(c / L::CPR, c % L::CPR)) = pa[i];
    }
#pragma unroll
    for (int i = 0; i < B_CH; ++i) {
      const int c = tid + i * kNT;
      const int o = L::off(c / L::CPR, c % L::CPR);
      *reinterpret_cast<uint4*>(base + L::A + o) = pb0[i];
      *reinterpret_cast<uint4*>(base + L::A + L::B + o) = pb1[i];
    }
  };

  v16f acc0[4][2], acc1[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        acc0[i][j][r] = 0.0f;
        acc1[i][j][r] = 0.0f;
      }

  const int nk = (K + BK - 1) / BK;
  if (nk > 0) {
    gload(0);
    lstore(0);
    __syncthreads();
  }
  for (int kt = 0; kt < nk; ++kt) {
    const bool more = kt + 1 < nk;
    if (more) gload(kt + 1);
    const uint8_t* base = smem + (kt & 1) * L::STAGE;
#pragma unroll
    for (int ks = 0; ks < BK / 64; ++ks) {
      const int c0 = ks * 4 + 2 * lg;  // this lane's two chunks of the 64-wide step
      v8i fa[4], fb0[2], fb1[2];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = wm * 128 + i * 32 + lr;
        fa[i] = make_frag(lds_read16(base, L::off(r, c0)), lds_read16(base, L::off(r, c0 + 1)));
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int r = wn * 64 + j * 32 + lr;
        fb0[j] = make_frag(lds_read16(base + L::A, L::off(r, c0)),
                           lds_read16(base + L::A, L::off(r, c0 + 1)));
        fb1[j] = make_frag(lds_read16(base + L::A + L::B, L::off(r, c0)),
                           lds_read16(base + L::A + L::B, L::off(r, c0 + 1)));
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          acc0[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
              fa[i], fb0[j], acc0[i][j], AF, BF, 0, 127, 0, 127);
          acc1[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
              fa[i], fb1[j], acc1[i][j], AF, BF, 0, 127, 0, 127);
        }
    }
    if (more) lstore((kt + 1) & 1);
    __syncthreads();
  }

  // ---- epilogue: scale, combine, store ----
  const float sa = *s_a;
  const float c0s = sa * *s_0;
  const float c1s = sa * *s_1;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int colw = wn * 64 + j * 32 + lr;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm * 128 + i * 32 + (r >> 2) * 8 + lg * 4 + (r & 3);
        if (row >= M) continue;
        OutT* orow = out + int64_t(row) * ldo;
        if constexpr (SPLIT) {
          const int ca = n0 + colw, cb = n1 + colw;
          if (ca < N) store_out<OutT>(orow + ca, acc0[i][j][r] * c0s + (bias ? bias[ca] : 0.0f));
          if (cb < N) store_out<OutT>(orow + cb, acc1[i][j][r] * c0s + (bias ? bias[cb] : 0.0f));
        } else {
          const int col = n0 + colw;
          if (col < N) {
            float v = acc0[i][j][r] * c0s + acc1[i][j][r] * c1s;
            if (bias) v += bias[col];
            store_out<OutT>(orow + col, v);
          }
        }
      }
    }
}

constexpr int kBK = 64;

template <int AF, int BF, bool SPLIT, typename OutT>
int launch_gemm(const uint8_t* a, int64_t lda, const uint8_t* b0, const uint8_t* b1, int64_t ldb,
                int m, int n, int k, const float* s_a, const float* s_0, const float* s_1,
                const float* bias, OutT* out, int64_t ldo, hipStream_t st) {
  const int tiles_m = (m + kBM - 1) / kBM;
  const int tn_w = SPLIT ? 2 * kBN : kBN;
  const int tiles_n = (n + tn_w - 1) / tn_w;
  const int smem = 2 * Lds<kBK>::STAGE;
  auto kern = gemm_nt_kernel<AF, BF, SPLIT, kBK, OutT>;
  static bool attr_set = false;
  if (!attr_set) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                            hipFuncAttributeMaxDynamicSharedMemorySize, smem) != hipSuccess)
      return TCFP_ERR_HIP;
    attr_set = true;
  }
  kern<<<tiles_m * tiles_n, kNT, smem, st>>>(a, b0, b1, m, n, k, lda, ldb, s_a, s_0, s_1, bias,
                                             out, ldo, tiles_m, tiles_n);
  return hipGetLastError() == hipSuccess ? TCFP_OK : TCFP_ERR_HIP;
}

template <bool SPLIT, typename OutT>
int dispatch_fmt(int a_fmt, int b_fmt, const uint8_t* a, int64_t lda, const uint8_t* b0,
                 const uint8_t* b1, int64_t ldb, int m, int n, int k, const float* s_a,
                 const float* s_0, const float* s_1, const float* bias, OutT* out, int64_t ldo,
                 hipStream_t st) {
#define TCFP_G(AF, BF) \
  launch_gemm<AF, BF, SPLIT, OutT>(a, lda, b0, b1, ldb, m, n, k, s_a, s_0, s_1, bias, out, ldo, st)
  if (a_fmt == TCFP_FP8_E4M3 && b_fmt == TCFP_FP8_E4M3) return TCFP_G(0, 0);
  if (a_fmt == TCFP_FP8_E5M2 && b_fmt == TCFP_FP8_E4M3) return TCFP_G(1, 0);
  if (a_fmt == TCFP_FP8_E4M3 && b_fmt == TCFP_FP8_E5M2) return TCFP_G(0, 1);
  if (a_fmt == TCFP_FP8_E5M2 && b_fmt == TCFP_FP8_E5M2) return TCFP_G(1, 1);
#undef TCFP_G
  return TCFP_ERR_DTYPE;
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

extern "C" int tcfp_dual_gemm(const uint8_t* a, int a_fmt, int64_t lda, const uint8_t* b_hi,
                              const uint8_t* b_lo, int b_fmt, int64_t ldb, int64_t m, int64_t n,
                              int64_t k, const float* s_a, const float* s_hi, const float* s_lo,
                              const float* bias, void* out, int out_dtype, int64_t ldo,
                              void* stream) {
  if (m < 0 || n < 0 || k < 0 || m > INT32_MAX || n > INT32_MAX || k > INT32_MAX)
    return TCFP_ERR_SHAPE;
  if (k % 16 != 0) return TCFP_ERR_SHAPE;
  if (lda < k || ldb < k || ldo < n) return TCFP_ERR_SHAPE;
  if (lda % 16 != 0 || ldb % 16 != 0) return TCFP_ERR_ALIGN;
  if (!al16(a) || !al16(b_hi) || (b_lo && !al16(b_lo))) return TCFP_ERR_ALIGN;
  if (!s_a || !s_hi || (b_lo && !s_lo)) return TCFP_ERR_SHAPE;
  if (out_dtype != TCFP_DTYPE_F32 && out_dtype != TCFP_DTYPE_BF16) return TCFP_ERR_DTYPE;
  if (m == 0 || n == 0) return TCFP_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int M = int(m), N = int(n), K = int(k);
  if (b_lo) {
    if (out_dtype == TCFP_DTYPE_F32)
      return dispatch_fmt<false, float>(a_fmt, b_fmt, a, lda, b_hi, b_lo, ldb, M, N, K, s_a, s_hi,
                                        s_lo, bias, static_cast<float*>(out), ldo, st);
    return dispatch_fmt<false, uint16_t>(a_fmt, b_fmt, a, lda, b_hi, b_lo, ldb, M, N, K, s_a, s_hi,
                                         s_lo, bias, static_cast<uint16_t*>(out), ldo, st);
  }
  if (out_dtype == TCFP_DTYPE_F32)
    return dispatch_fmt<true, float>(a_fmt, b_fmt, a, lda, b_hi, b_hi, ldb, M, N, K, s_a, s_hi,
                                     s_hi, bias, static_cast<float*>(out), ldo, st);
  return dispatch_fmt<true, uint16_t>(a_fmt, b_fmt, a, lda, b_hi, b_hi, ldb, M, N, K, s_a, s_hi,
                                      s_hi, bias, static_cast<uint16_t*>(out), ldo, st);
}
