// Shared device helpers for the TCFP-12 HIP kernels (gfx950 / CDNA4).
//
// Numerics follow the reference's torch semantics bit-for-bit:
//   * FP8 casts are round-to-nearest-even (torch `.to(float8_*)`),
//   * per-tensor scales are `reciprocal(amax) * FP8_MAX` in the input dtype
//     (torch `Tensor.__rtruediv__`, reference tcfp/core.py:100-101),
//   * block exponents are `ceil(log2(amax / FP8_MAX))` as a correctly
//     rounded fp32 log2 evaluates it (reference tcfp/kernels.py:253-260).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/tcfp_hip.h"

#define TCFP_DEV __device__ __forceinline__

namespace tcfp {

constexpr float kE4M3Max = 448.0f;
constexpr float kE5M2Max = 57344.0f;

TCFP_DEV float fp8_max(int fmt) { return fmt == TCFP_FP8_E5M2 ? kE5M2Max : kE4M3Max; }

// HIP launch limit along x: gridDim.x * blockDim.x must stay below 2^32.
inline bool grid_x_fits(int64_t blocks, int threads) {
  return blocks >= 0 && blocks <= int64_t(UINT32_MAX) / threads;
}

// ---- column sums (bias gradients) -----------------------------------------
// Every column sum this library computes of a [rows, cols] fp32 tensor x
// (the producers: the tiled quantisation pass and the dgrad GEMM's GELU
// epilogue) has one order, so that either producer gives the same bits:
//  1. per 64-row group q (rows 64q ... 64q + 63, missing rows +0) and column
//     c: y[l] = x[64q + l][c] + x[64q + 32 + l][c] for l < 32, then halving
//     folds y[l] = y[l] + y[l + d] for l < d, d = 16, 8, 4, 2, 1, giving
//     P[q][c] = y[0];
//  2. the finalising pass (quant.hip) adds the P[q][c] over q.
constexpr int kColGroup = 64;
constexpr int kColHalf = kColGroup / 2;

// ---- shared between the GEMM and quantisation sources (quant.hip) --------
// Slots of per-workgroup partial maxima the per-tensor reduction workspace
// holds (its first member, at offset 0).
int max_parts();
// Per-tensor quantisation of x whose partial maxima (|value| as float bits,
// NaN above inf) a producer already wrote to the first pre_g workspace
// slots: the quantising pass of tcfp_quantize_per_tensor, with gelu_in (x
// is fp32 h, the values are gelu(h)) and col_sum (column sums per 128-row
// tile in cs_ws, then over the tiles) as in that file.
int quantize_with_parts(const void* x, int x_dtype, int64_t rows, int64_t cols, int fp8_fmt,
                        uint8_t* q, uint8_t* q_t, float* inv_out, void* workspace,
                        float* col_sum, float* cs_ws, void* stream, int pre_g, bool gelu_in);
// col_sum[c] = the sum over the first `groups` rows of cs_ws ([groups, cols]
// per-group partials) in the finalising order.
int colsum_finalize(const float* cs_ws, int64_t groups, int64_t cols, float* col_sum,
                    void* stream);
// gelu(h) quantised per tensor (as tcfp_gelu_quantize_per_tensor) with the
// amax from the GELU amax rule's keys a producer of h wrote, one (int max,
// uint max) pair per producer workgroup, at keys[2 i], keys[2 i + 1],
// i < n_keys (keys must not overlap the workspace's first slots).  When the
// rule does not apply, a full GELU amax pass over h runs in its place (on
// the device: the launch sequence is the same).  act (gelu(h)) and dgelu
// (the derivative factor of gelu_and_deriv) are written when not null.
// cols % 8 == 0.
int gelu_quantize_from_keys(const float* h, int64_t rows, int64_t cols, int fp8_fmt, float* act,
                            float* dgelu, uint8_t* q, uint8_t* q_t, float* inv_out,
                            void* workspace, const uint32_t* keys, int n_keys, void* stream);
// out = a * b elementwise and the per-tensor quantisation of out with its
// column sums (tcfp_quantize_per_tensor_colsum, col_sum may be null): the
// GELU backward from its saved derivative factor (a = dy, b = dgelu).  out
// may be a.  cols % 8 == 0.
int mul_quantize_colsum(const float* a, const float* b, int64_t rows, int64_t cols, int fp8_fmt,
                        float* out, uint8_t* q, uint8_t* q_t, float* inv_out, float* col_sum,
                        void* workspace, float* cs_ws, void* stream);

// ---------------------------------------------------------------------------
// bfloat16
// ---------------------------------------------------------------------------
TCFP_DEV float bf16_to_f32(uint16_t h) { return __uint_as_float(uint32_t(h) << 16); }

TCFP_DEV uint16_t f32_to_bf16_rne(float x) {
  uint32_t b = __float_as_uint(x);
  if ((b & 0x7FFFFFFFu) > 0x7F800000u) return uint16_t((b >> 16) | 0x40u);
  b += 0x7FFFu + ((b >> 16) & 1u);
  return uint16_t(b >> 16);
}

TCFP_DEV float round_bf16(float x) { return bf16_to_f32(f32_to_bf16_rne(x)); }

// ---------------------------------------------------------------------------
// FP8 encode / decode (software, exact).  `sat` selects saturation to the
// largest finite code instead of torch's overflow codes (E4M3FN: NaN 0x7F,
// E5M2: inf 0x7C); the reference clamps before casting, so both agree on
// its inputs.
// ---------------------------------------------------------------------------
TCFP_DEV uint32_t f32_to_e4m3(float x, bool sat = false) {
  uint32_t b = __float_as_uint(x);
  uint32_t s = (b >> 24) & 0x80u;
  uint32_t m = b & 0x7FFFFFFFu;
  if (m > 0x7F800000u) return s | 0x7Fu;
  uint32_t q;
  if (m < 0x3C800000u) {  // below 2^-6: multiples of 2^-9
    q = uint32_t(__float2int_rn(__uint_as_float(m) * 512.0f));
  } else {
    uint32_t r = m + 0x7FFFFu + ((m >> 20) & 1u);
    q = (r >> 20) - (120u << 3);
    uint32_t top = sat ? 0x7Eu : 0x7Fu;
    q = q > top ? top : q;
  }
  return s | q;
}

TCFP_DEV uint32_t f32_to_e5m2(float x, bool sat = false) {
  uint32_t b = __float_as_uint(x);
  uint32_t s = (b >> 24) & 0x80u;
  uint32_t m = b & 0x7FFFFFFFu;
  if (m > 0x7F800000u) return s | 0x7Fu;
  uint32_t q;
  if (m < 0x38800000u) {  // below 2^-14: multiples of 2^-16
    q = uint32_t(__float2int_rn(__uint_as_float(m) * 65536.0f));
  } else {
    uint32_t r = m + 0xFFFFFu + ((m >> 21) & 1u);
    q = (r >> 21) - (112u << 2);
    uint32_t top = sat ? 0x7Bu : 0x7Cu;
    q = q > top ? top : q;
  }
  return s | q;
}

template <int FMT>
TCFP_DEV uint32_t f32_to_fp8(float x, bool sat = false) {
  if constexpr (FMT == TCFP_FP8_E5M2) return f32_to_e5m2(x, sat);
  else return f32_to_e4m3(x, sat);
}

// Software decoders (exact, from the OCP FP8 definitions): the reference
// the hardware decoders below are checked against, code by code.
TCFP_DEV float sw_e4m3_to_f32(uint32_t c) {
  uint32_t s = (c & 0x80u) << 24;
  uint32_t e = (c >> 3) & 0xFu, m = c & 7u;
  uint32_t mag;
  if (e == 0) mag = __float_as_uint(float(m) * 0.001953125f);  // m * 2^-9
  else if (e == 15 && m == 7) mag = 0x7FC00000u;
  else mag = ((e + 120u) << 23) | (m << 20);
  return __uint_as_float(s | mag);
}

TCFP_DEV float sw_e5m2_to_f32(uint32_t c) {
  uint32_t s = (c & 0x80u) << 24;
  uint32_t e = (c >> 2) & 0x1Fu, m = c & 3u;
  uint32_t mag;
  if (e == 0) mag = __float_as_uint(float(m) * 1.52587890625e-05f);  // m * 2^-16
  else if (e == 31) mag = m ? 0x7FC00000u : 0x7F800000u;
  else mag = ((e + 112u) << 23) | (m << 21);
  return __uint_as_float(s | mag);
}

template <int FMT>
TCFP_DEV float sw_fp8_to_f32(uint32_t c) {
  if constexpr (FMT == TCFP_FP8_E5M2) return sw_e5m2_to_f32(c);
  else return sw_e4m3_to_f32(c);
}

// Hardware decoders (v_cvt_f32_fp8 / v_cvt_f32_bf8, byte 0 of c): one
// instruction.  Every FP8 value is exact in fp32; the GPU self-test checks
// all 256 codes of both formats against the software decoders (NaN codes
// decode to a NaN in both).
TCFP_DEV float e4m3_to_f32(uint32_t c) { return __builtin_amdgcn_cvt_f32_fp8(int(c), 0); }
TCFP_DEV float e5m2_to_f32(uint32_t c) { return __builtin_amdgcn_cvt_f32_bf8(int(c), 0); }

template <int FMT>
TCFP_DEV float fp8_to_f32(uint32_t c) {
  if constexpr (FMT == TCFP_FP8_E5M2) return e5m2_to_f32(c);
  else return e4m3_to_f32(c);
}

// Hardware conversion of four clamped, finite floats (gfx950 OCP FP8,
// round-to-nearest-even).  Bit-identity with the software path above on
// every finite in-range float32 is checked on the GPU by the test suite.
template <int FMT>
TCFP_DEV uint32_t cvt4_fp8(float a, float b, float c, float d) {
  int r;
  if constexpr (FMT == TCFP_FP8_E5M2) {
    r = __builtin_amdgcn_cvt_pk_bf8_f32(a, b, 0, false);
    r = __builtin_amdgcn_cvt_pk_bf8_f32(c, d, r, true);
  } else {
    r = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
    r = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, r, true);
  }
  return uint32_t(r);
}

template <int FMT>
TCFP_DEV uint32_t sw4_fp8(float a, float b, float c, float d) {
  return f32_to_fp8<FMT>(a) | (f32_to_fp8<FMT>(b) << 8) | (f32_to_fp8<FMT>(c) << 16) |
         (f32_to_fp8<FMT>(d) << 24);
}

// ---------------------------------------------------------------------------
// ceil(log2(q)) as torch evaluates it for positive normal fp32 q:
// exact integer logic reproducing a correctly rounded fp32 log2 followed by
// ceil.  For q = 2^k (1 + j 2^-23) the rounded log2 equals k exactly when
// j <= J(p), where p is the binade exponent of the fp32 numbers just past k
// toward k + log2(1+f); J = floor(ln2 * 2^(p-1)) = {0,0,1,2,5,11,22}.
// Subnormal q returns -127 (callers clamp at -126).
// ---------------------------------------------------------------------------
TCFP_DEV int ceil_log2_f32(float q) {
  // (written without early returns: every case is a select, so the
  // compiler emits no divergent branches where lanes hold different q)
  const uint32_t b = __float_as_uint(q);
  const int ef = int((b >> 23) & 0xFFu);
  const int k = ef - 127;
  const uint32_t j = b & 0x7FFFFFu;
  const uint32_t a = uint32_t(k < 0 ? -k : k);
  int p = a != 0u ? 31 - __clz(a) : 0;
  if (k < 0 && (a & (a - 1u)) == 0u) p -= 1;
  const uint64_t table = 0x16'0B'05'02'01'00'00ull;  // J(p) bytes, p = 0..6
  const uint32_t jmax = p <= 0 ? 0u : uint32_t((table >> (8 * p)) & 0xFFu);
  return ef == 0 ? -127 : k + (j > jmax ? 1 : 0);
}

// Block exponent rule: max(ceil(log2(max(amax,1e-12) / FP8_MAX)), -126).
TCFP_DEV int block_exponent(float amax, float fmax) {
  float a = fmaxf(amax, 1e-12f);
  int e = ceil_log2_f32(__fdiv_rn(a, fmax));
  return e < -126 ? -126 : e;
}

// 2^e as float for e in [-149, 127].
TCFP_DEV float exp2i(int e) {
  if (e >= -126) return __uint_as_float(uint32_t(e + 127) << 23);
  return __uint_as_float(1u << (e + 149));
}

// |v| as float bits: unsigned order is the order of |v|, NaN above inf (the
// encoding of every partial maximum).
TCFP_DEV uint32_t absbits(float v) { return __float_as_uint(v) & 0x7FFFFFFFu; }
TCFP_DEV uint32_t umax(uint32_t a, uint32_t b) { return a > b ? a : b; }

// torch.clamp semantics: NaN passes through.
TCFP_DEV float clampf(float v, float mx) { return v > mx ? mx : (v < -mx ? -mx : v); }

// Max over each group of L consecutive lanes (L a power of two <= 32),
// returned to every lane of the group.  DPP permutations inside a row of 16
// lanes (quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror,
// row_mirror: after each step every lane holds the max of a group twice as
// large) need no index arithmetic; the 32-lane step is a ds_swizzle with
// xor mask 16.  Every lane of the wave executes the reduction.
template <int L>
TCFP_DEV uint32_t seg_umax(uint32_t m) {
  if constexpr (L >= 2) m = umax(m, uint32_t(__builtin_amdgcn_update_dpp(0, int(m), 0xB1, 0xF, 0xF, false)));
  if constexpr (L >= 4) m = umax(m, uint32_t(__builtin_amdgcn_update_dpp(0, int(m), 0x4E, 0xF, 0xF, false)));
  if constexpr (L >= 8) m = umax(m, uint32_t(__builtin_amdgcn_update_dpp(0, int(m), 0x141, 0xF, 0xF, false)));
  if constexpr (L >= 16) m = umax(m, uint32_t(__builtin_amdgcn_update_dpp(0, int(m), 0x140, 0xF, 0xF, false)));
  if constexpr (L >= 32) m = umax(m, uint32_t(__builtin_amdgcn_ds_swizzle(int(m), 0x401F)));
  static_assert(L >= 1 && L <= 32 && (L & (L - 1)) == 0, "segment of 1..32 lanes");
  return m;
}


// ---------------------------------------------------------------------------
// GELU
// ---------------------------------------------------------------------------
// GELU (erf form) exactly as torch evaluates it on fp32 tensors: forward
// x * 0.5 * (1 + erf(x * sqrt(1/2))), every operation rounded on its own
// (every file that includes this header is built without contraction); backward
// dy * (cdf + x * pdf) with cdf = 0.5 * (1 + erf(x * sqrt(1/2))),
// pdf = exp(-0.5 * x * x) * (2/sqrt(pi) * sqrt(1/2) * 0.5), the last
// product and sum as one fused multiply-add.  The constants are the
// double-precision products rounded once to fp32.  A GPU test holds both
// bitwise equal to torch.nn.functional.gelu and its gradient.
constexpr float kSqrtHalf = float(0.70710678118654752440);
constexpr float kGeluBeta = float(1.12837916709551257390 * 0.70710678118654752440 * 0.5);
TCFP_DEV float gelu_f32(float x) { return x * 0.5f * (1.0f + erff(x * kSqrtHalf)); }
TCFP_DEV float gelu_bwd_f32(float x, float dy) {
  const float cdf = 0.5f * (1.0f + erff(x * kSqrtHalf));
  const float pdf = expf(-0.5f * x * x) * kGeluBeta;
  return dy * __builtin_fmaf(x, pdf, cdf);
}
// gelu(x) and the derivative factor d(x) = cdf + x * pdf of gelu_bwd_f32,
// sharing the erf: gelu_bwd_f32(x, dy) == dy * d(x) bit for bit.
TCFP_DEV void gelu_and_deriv(float x, float& g, float& d) {
  const float e = erff(x * kSqrtHalf);
  g = x * 0.5f * (1.0f + e);
  const float cdf = 0.5f * (1.0f + e);
  const float pdf = expf(-0.5f * x * x) * kGeluBeta;
  d = __builtin_fmaf(x, pdf, cdf);
}

// Keys of the GELU amax rule.  A producer of h tracks, over its values,
// the max of the float bits as int32 (the largest h >= +0, or INT32_MIN when
// every value is negative or -0; +NaN sorts above +inf) and as uint32
// (>= 0xFF800000 exactly when some value is -inf or a negative NaN).  When
// gelu is non-decreasing on [+0, +inf] and |gelu| stays below a bound T on
// the negative numbers (both checked once per device by quant.hip), the
// max |gelu(h)| is gelu(max h) whenever that is finite, not NaN and >= T.
constexpr uint32_t kGeluKeyNegNanInf = 0xFF800000u;
constexpr uint32_t kGeluKeyPosInf = 0x7F800000u;

// ---------------------------------------------------------------------------
// Philox4x32-10 (Salmon, Moraes, Dror, Shaw: "Parallel random numbers: as
// easy as 1, 2, 3", SC'11).  Counter-based: each element draws from its own
// (index, offset) counter, so results do not depend on launch shape.
// ---------------------------------------------------------------------------
struct u32x4 { uint32_t x, y, z, w; };

TCFP_DEV u32x4 philox4x32_10(u32x4 c, uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    uint64_t p0 = uint64_t(0xD2511F53u) * c.x;
    uint64_t p1 = uint64_t(0xCD9E8D57u) * c.z;
    u32x4 n;
    n.x = uint32_t(p1 >> 32) ^ c.y ^ k0;
    n.y = uint32_t(p1);
    n.z = uint32_t(p0 >> 32) ^ c.w ^ k1;
    n.w = uint32_t(p0);
    c = n;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  return c;
}

TCFP_DEV float u32_to_unit(uint32_t v) { return float(v >> 8) * 5.9604644775390625e-08f; }

// ---------------------------------------------------------------------------
// Reductions (wave64)
// ---------------------------------------------------------------------------
TCFP_DEV float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// |x| max that propagates NaN like torch.max.
TCFP_DEV float nanmax(float a, float b) {
  return (a != a || b != b) ? __uint_as_float(0x7FC00000u) : fmaxf(a, b);
}

TCFP_DEV float wave_nanmax(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = nanmax(v, __shfl_xor(v, o, 64));
  return v;
}

}  // namespace tcfp
