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

// ===========================================================================
// Main kernel: LDS double buffer filled by direct global->LDS DMA
// ===========================================================================
//
// Same 256 x (2 x 128) workgroup tile and 2 x 2 wave grid as above, with
// the choices that measured fastest on gfx950:
//  * Operand tiles go from HBM/L2 straight into LDS with
//    `buffer_load_dwordx4 ... lds` (no VGPR staging, no LDS store
//    instructions).  A stage covers 128 K columns, so every row
//    contributes one full 128-byte cache line per stage: fetching half
//    lines (64 K columns) halves the L2->LDS rate (27 vs 57 B/clk/CU
//    measured).  Two 64 KiB stages fill 128 KiB of the 160 KiB LDS.
//  * Each stage is two MFMA sub-steps of 64 K.  Fragments live in two
//    register sets: while the MFMAs of one sub-step run, the fragments of
//    the next are read from LDS, one 16-byte LDS read per MFMA.  The DMA
//    of stage t + 2 is issued half-way through stage t, as soon as every
//    wave has read its last fragments of stage t, so it has a full stage
//    of MFMA time to land.
//  * Buffer addressing gives free bounds handling: rows past M/N and K
//    chunks past K are given an offset beyond the descriptor's range and
//    the hardware returns zeros, so no tail masking is needed in the loop.
//  * The MFMA "A" operand is the weight tile and "B" the activation tile,
//    so an accumulator lane holds four consecutive output columns of one
//    row: the epilogue writes 8/16-byte vectors instead of 2-byte scalars.
//
// The DMA is issued from inline assembly: the compiler's wait-count pass
// does not know these writes do not alias the LDS reads of the other
// buffer and would otherwise drain all loads before every LDS read.  Wait
// counts for the DMA are therefore explicit (s_waitcnt before the barrier).
//
// Stage layout (512 rows of 128 bytes): rows 0-255 activation rows m0..,
// rows 256-383 slot-0 weight rows, rows 384-511 slot-1 weight rows.  The
// eight 16-byte chunks of a row are permuted by swz(row) = (row >> 1) & 7,
// which makes the MFMA operand reads (32 consecutive rows, same chunk)
// bank-conflict free on the 64-bank (256 B/clk) LDS.

typedef int v4i __attribute__((ext_vector_type(4)));
#define TCFP_LDS __attribute__((address_space(3)))

constexpr int kSK = 128;                 // K columns per stage
constexpr int kRowB = kSK;               // bytes per stage row
constexpr int kStageBytes = 512 * kRowB; // 64 KiB
constexpr uint32_t kOob = 0x80000000u;   // beyond every descriptor's range

TCFP_DEV int swz(int row) { return (row >> 1) & 7; }

TCFP_DEV v4i make_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  v4i r;
  r[0] = int(uint32_t(a));
  r[1] = int(uint32_t(a >> 32) & 0xFFFFu);  // stride 0: raw byte addressing
  r[2] = int(bytes);                        // num_records: bytes in range
  r[3] = 0x00020000;                        // gfx9 raw-buffer data format word
  return r;
}

// 64 lanes x 16 bytes from rsrc + voff + soff into LDS [lds, lds + 1024).
TCFP_DEV void dma16(v4i rsrc, uint32_t voff, uint32_t soff, uint32_t lds) {
  asm volatile("buffer_load_dwordx4 %0, %1, %2 offen lds"
               :
               : "v"(voff), "s"(rsrc), "s"(soff), "{m0}"(lds)
               : "memory");
}

template <typename OutT>
TCFP_DEV void store4(OutT* p, float a, float b, float c, float d);
template <>
TCFP_DEV void store4<float>(float* p, float a, float b, float c, float d) {
  *reinterpret_cast<float4*>(p) = make_float4(a, b, c, d);
}
template <>
TCFP_DEV void store4<uint16_t>(uint16_t* p, float a, float b, float c, float d) {
  // v_cvt_pk_bf16_f32: round-to-nearest-even, two values per instruction
  typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
  const bf2 lo = {(__bf16)a, (__bf16)b};
  const bf2 hi = {(__bf16)c, (__bf16)d};
  *reinterpret_cast<uint2*>(p) =
      make_uint2(__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi));
}

// Scheduling pattern for one sub-step: NMF MFMAs with NRD LDS reads spread
// evenly between them (sched_group_barrier masks: 0x008 MFMA, 0x100 DS read).
template <int NMF, int NRD, int Q>
TCFP_DEV void interleave_mfma_lds() {
  if constexpr (Q < NMF) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    constexpr int rd = (Q + 1) * NRD / NMF - Q * NRD / NMF;
    if constexpr (rd > 0) __builtin_amdgcn_sched_group_barrier(0x100, rd, 0);
    interleave_mfma_lds<NMF, NRD, Q + 1>();
  }
}

// NW = 4: one wave per SIMD, 2 x 2 wave grid, 128 x 64 (x2 slots) per wave.
// NW = 8: two waves per SIMD, 4 x 2 wave grid, 64 x 64 (x2 slots) per wave;
//         half the accumulators per wave, so two waves fit one SIMD and the
//         MFMA pipe keeps issuing while the other wave waits.
template <int AF, int BF, bool SPLIT, typename OutT, int NW>
__global__ __launch_bounds__(NW * 64, 1) void gemm_nt_dma_kernel(
    const uint8_t* __restrict__ A, const uint8_t* __restrict__ B0, const uint8_t* __restrict__ B1,
    int M, int N, int K, int64_t lda, int64_t ldb, const float* __restrict__ s_a,
    const float* __restrict__ s_0, const float* __restrict__ s_1, const float* __restrict__ bias,
    OutT* __restrict__ out, int64_t ldo, int tiles_m, int tiles_n) {
  constexpr int WM = NW / 2;        // wave rows
  constexpr int TMW = kBM / WM;     // activation rows per wave (128 or 64)
  constexpr int MB = TMW / 32;      // 32-row m-blocks per wave (4 or 2)
  constexpr int RPW = 512 / NW;     // stage rows DMA'd by each wave (128 or 64)
  constexpr int DI = RPW / 8;       // 1 KiB DMA instructions per wave and stage
  __shared__ __align__(16) uint8_t lds[2 * kStageBytes];

  // ---- tile mapping (XCD-aware, grouped; as in gemm_nt_kernel) ----
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
  const int n1 = SPLIT ? n0 + kBN : n0;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int lr = lane & 31, lg = lane >> 5;

  // ---- this wave's DMA source: stage rows [wave*RPW, +RPW) lie in one of
  // the activation (0-255), slot-0 (256-383) or slot-1 (384-511) regions
  const int srow0 = wave * RPW;
  const uint8_t* src;
  int64_t ld;
  int rows_left, row_base;
  if (srow0 < 256) {
    src = A + int64_t(m0) * lda; ld = lda; rows_left = min(M - m0, kBM); row_base = srow0;
  } else if (srow0 < 384) {
    src = B0 + int64_t(n0) * ldb; ld = ldb; rows_left = min(N - n0, kBN); row_base = srow0 - 256;
  } else {
    src = B1 + int64_t(n1) * ldb; ld = ldb; rows_left = min(N - n1, kBN); row_base = srow0 - 384;
  }
  const uint32_t nrec = rows_left > 0 ? uint32_t(int64_t(rows_left - 1) * ld + K) : 0u;
  const v4i rsrc = make_rsrc(src, nrec);
  // Instruction i fills stage rows srow0 + i*8 .. +8 (1 KiB); lane writes row
  // +lane/8 at physical chunk lane%8.  srow0 is a multiple of 64, so the
  // logical chunk depends on i only through i's low bit.
  const int chunk0 = (lane & 7) ^ swz(lane >> 3);        // even i
  const int chunk1 = (lane & 7) ^ swz(8 + (lane >> 3));  // odd i
  uint32_t voff[DI];
#pragma unroll
  for (int i = 0; i < DI; ++i) {
    const int r = row_base + i * 8 + (lane >> 3);
    const int c = (i & 1) ? chunk1 : chunk0;
    voff[i] = r < rows_left ? uint32_t(int64_t(r) * ld + c * 16) : kOob;
  }
  const uint32_t lds_base =
      uint32_t(reinterpret_cast<uintptr_t>((TCFP_LDS uint8_t*)lds)) + uint32_t(srow0) * kRowB;
  const int nt = (K + kSK - 1) / kSK;
  const int krem = K - (nt - 1) * kSK;  // valid K columns of the last stage

  // DMA of stage t (K columns t*128 ..) into buffer t & 1.  Stages past the
  // end are issued as all-out-of-range loads (zeros into a buffer nobody
  // reads again): the issue stays branch-free, so the loop body is a single
  // basic block and the compiler cannot sink MFMAs across the barrier.
  auto issue = [&](int t) {
    const uint32_t dst = lds_base + uint32_t(t & 1) * kStageBytes;
    const bool live = t < nt;
    const uint32_t soff = uint32_t(live ? t : 0) * kSK;
    const bool last = t == nt - 1;
#pragma unroll
    for (int i = 0; i < DI; ++i) {
      const int c = (i & 1) ? chunk1 : chunk0;
      dma16(rsrc, (!live || (last && c * 16 >= krem)) ? kOob : voff[i], soff, dst + i * 1024);
    }
  };

  // ---- per-lane LDS read offsets: sub-step h, 16-byte half q of a fragment
  int ro[2][2];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int q = 0; q < 2; ++q) ro[h][q] = lr * kRowB + (((4 * h + 2 * lg + q) ^ swz(lr)) << 4);

  v16f acc[2][2][MB];  // [slot][n-block][m-block]
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[s][j][i][r] = 0.0f;

  // Fragments of sub-step h of stage t: [0..3] weights (slot, n-block),
  // [4..4+MB) activations (m-block).
  auto read_frags = [&](v8i* f, int t, int h) {
    const uint8_t* st = lds + (t & 1) * kStageBytes;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int rb = (256 + (q >> 1) * 128 + wn * 64 + (q & 1) * 32) * kRowB;
      f[q] = make_frag(lds_read16(st, rb + ro[h][0]), lds_read16(st, rb + ro[h][1]));
    }
#pragma unroll
    for (int i = 0; i < MB; ++i) {
      const int rb = (wm * TMW + i * 32) * kRowB;
      f[4 + i] = make_frag(lds_read16(st, rb + ro[h][0]), lds_read16(st, rb + ro[h][1]));
    }
  };
  auto mfmas = [&](const v8i* f) {
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        acc[q >> 1][q & 1][i] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
            f[q], f[4 + i], acc[q >> 1][q & 1][i], BF, AF, 0, 127, 0, 127);
  };
  // 4*MB MFMAs and 2*(4+MB) LDS reads per sub-step: spread the reads evenly
  auto interleave = [&]() { interleave_mfma_lds<4 * MB, 2 * (4 + MB), 0>(); };
  // All DMA issued so far has landed and every wave's LDS reads are done
  // (gfx9 s_waitcnt: vmcnt bits [3:0] and [15:14], expcnt [6:4], lgkmcnt [11:8]).
  // sched_barrier(0) keeps the scheduler from moving MFMAs across it: MFMAs
  // touch no memory, so without it they drift past the barrier and the LDS
  // reads before it are left with nothing to hide behind.
  auto sync_all = [&]() {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0), expcnt untouched
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  };

  v8i f0[4 + MB], f1[4 + MB];
  if (nt > 0) {
    issue(0);
    if (nt > 1) issue(1);
    // wait for stage 0 only: stage 1's DI loads may stay in flight
    if (nt > 1) __builtin_amdgcn_s_waitcnt((DI & 15) | (7 << 4) | ((DI >> 4) << 14));
    else __builtin_amdgcn_s_waitcnt(0x0070);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    read_frags(f0, 0, 0);
  }
  for (int t = 0; t < nt; ++t) {
    // sub-step 0 of stage t; fragments of sub-step 1 stream in
    read_frags(f1, t, 1);
    mfmas(f0);
    interleave();
    // stage t + 1 landed, every wave has its stage-t fragments: refill t's buffer
    sync_all();
    issue(t + 2);
    __builtin_amdgcn_sched_barrier(0);
    // sub-step 1 of stage t; fragments of stage t + 1 sub-step 0 stream in
    // (after the last stage they read a stale buffer and are never used)
    read_frags(f0, t + 1, 0);
    mfmas(f1);
    interleave();
  }

  // ---- epilogue -----------------------------------------------------------
  // A lane holds rows m, columns n..n+3 of each 32x32 block: storing that
  // directly writes 16 bytes into each of 32 rows per instruction.  Instead
  // each wave stages its 64-column tile (per slot) through its own LDS
  // region and stores whole rows: 8 (bf16) or 4 (fp32) rows of 128/256
  // bytes per instruction, i.e. full cache lines.
  constexpr int EB = int(sizeof(OutT));      // output element bytes
  constexpr int RB = 64 * EB;                // bytes of one staged tile row
  constexpr int CPR = RB / 16;               // 16-byte chunks per row (8 / 16)
  constexpr int RPI = 64 / CPR;              // rows per store instruction
  uint8_t* eps = lds + wave * (TMW * RB);    // this wave's staging region
  const float sa = *s_a;
  const float c0s = sa * *s_0;
  const float c1s = SPLIT ? c0s : sa * *s_1;
  const bool vec = (ldo % (16 / EB)) == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0;
  // every wave is done with the operand buffers before they are reused
  __builtin_amdgcn_s_waitcnt(0x0070);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
#pragma unroll
  for (int s = 0; s < (SPLIT ? 2 : 1); ++s) {
    const int nb = (s ? n1 : n0) + wn * 64;  // first output column of this tile
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int row = i * 32 + lr, col = j * 32 + g * 8 + lg * 4;
          float v[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int r = g * 4 + q;
            v[q] = SPLIT ? acc[s][j][i][r] * c0s : acc[0][j][i][r] * c0s + acc[1][j][i][r] * c1s;
          }
          if (bias) {
#pragma unroll
            for (int q = 0; q < 4; ++q) v[q] += nb + col + q < N ? bias[nb + col + q] : 0.0f;
          }
          // 16-byte chunk index within the row, XOR-permuted by row
          const int byte = col * EB;
          const int chunk = (byte >> 4) ^ (row & (CPR - 1));
          store4<OutT>(reinterpret_cast<OutT*>(eps + row * RB + chunk * 16 + (byte & 15)), v[0],
                       v[1], v[2], v[3]);
        }
    asm volatile("" ::: "memory");
#pragma unroll
    for (int it = 0; it < TMW / RPI; ++it) {
      const int row = it * RPI + lane / CPR, cl = lane % CPR;
      const uint4 d = *reinterpret_cast<const uint4*>(eps + row * RB + ((cl ^ (row & (CPR - 1))) * 16));
      const int m = m0 + wm * TMW + row;
      const int n = nb + cl * (16 / EB);
      if (m < M) {
        OutT* o = out + int64_t(m) * ldo + n;
        if (vec && n + 16 / EB <= N) {
          *reinterpret_cast<uint4*>(o) = d;
        } else {
          const OutT* e = reinterpret_cast<const OutT*>(&d);
#pragma unroll
          for (int q = 0; q < 16 / EB; ++q)
            if (n + q < N) o[q] = e[q];
        }
      }
    }
    asm volatile("" ::: "memory");
  }
}

// Largest byte span any DMA descriptor may cover (offsets are 32-bit and
// the out-of-range sentinel must stay beyond every span).
#ifndef TCFP_DMA_WAVES
#define TCFP_DMA_WAVES 8
#endif
constexpr int kDmaWaves = TCFP_DMA_WAVES;

constexpr int64_t kMaxSpan = (int64_t(1) << 31) - (int64_t(1) << 20);

template <int AF, int BF, bool SPLIT, typename OutT>
int launch_gemm(const uint8_t* a, int64_t lda, const uint8_t* b0, const uint8_t* b1, int64_t ldb,
                int m, int n, int k, const float* s_a, const float* s_0, const float* s_1,
                const float* bias, OutT* out, int64_t ldo, hipStream_t st) {
  const int tiles_m = (m + kBM - 1) / kBM;
  const int tn_w = SPLIT ? 2 * kBN : kBN;
  const int tiles_n = (n + tn_w - 1) / tn_w;
  const bool dma_ok = int64_t(kBM) * lda + k < kMaxSpan && int64_t(kBN) * ldb + k < kMaxSpan &&
                      (bias == nullptr || (reinterpret_cast<uintptr_t>(bias) & 15) == 0);
  if (dma_ok) {
    gemm_nt_dma_kernel<AF, BF, SPLIT, OutT, kDmaWaves><<<tiles_m * tiles_n, kDmaWaves * 64, 0, st>>>(
        a, b0, b1, m, n, k, lda, ldb, s_a, s_0, s_1, bias, out, ldo, tiles_m, tiles_n);
    return hipGetLastError() == hipSuccess ? TCFP_OK : TCFP_ERR_HIP;
  }
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
