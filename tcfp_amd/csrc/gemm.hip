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
// Tiling (gemm_nt_dma_kernel below): a workgroup owns a BM x BN output
// tile per weight slot; per 128-column K stage the activation tile is
// brought into LDS once by direct global->LDS DMA and shared by the two
// weight slots (W_hi and W_lo) -- the dual GEMM is a single GEMM over
// [W_hi; W_lo] whose two accumulator halves meet in the epilogue.  Waves run
// v_mfma_scale_f32_32x32x64_f8f6f4 on fragments read from XOR-swizzled LDS
// rows (bank-conflict free).  In single-GEMM mode the two slots hold
// adjacent column halves of one 2*BN-wide tile.
//
// Workgroup -> tile mapping is XCD-aware: the dispatcher places workgroup b
// on XCD b % 8, so workgroups are renumbered to give each XCD a contiguous
// run of tiles, grouped 4 tile-rows deep, which keeps an XCD's A and B
// panels resident in its own L2.
#include <algorithm>
#include <type_traits>

#include "common.h"

using namespace tcfp;

namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

TCFP_DEV uint4 lds_read16(const uint8_t* base, int off) {
  return *reinterpret_cast<const uint4*>(base + off);
}

TCFP_DEV v8i make_frag(uint4 lo, uint4 hi) {
  v8i f;
  f[0] = int(lo.x); f[1] = int(lo.y); f[2] = int(lo.z); f[3] = int(lo.w);
  f[4] = int(hi.x); f[5] = int(hi.y); f[6] = int(hi.z); f[7] = int(hi.w);
  return f;
}


// ===========================================================================
// Main kernel: LDS double buffer filled by direct global->LDS DMA
// ===========================================================================
//
// A workgroup owns a BM (activation rows) x BN (weight rows) output tile
// and stages, per 128-column K step, BM activation rows and BN rows of each
// of two weight "slots" (W_hi and W_lo for the dual GEMM; adjacent column
// halves of one 2*BN-wide tile for a single GEMM).  Waves form a
// (NW/2) x 2 grid.  Two shapes are built:
//   BM = 256, BN = 128, 8 waves  -- one workgroup per CU, 128 KiB of LDS;
//   BM = 128, BN =  64, 4 waves  -- two workgroups per CU, so one
//       workgroup's epilogue overlaps the other's main loop; used when the
//       large tile would leave CUs idle (e.g. the wgrad GEMMs, whose
//       outputs are small and whose K is the token count).
// Choices that measured fastest on gfx950:
//  * Operand tiles go from HBM/L2 straight into LDS with
//    `buffer_load_dwordx4 ... lds` (no VGPR staging, no LDS store
//    instructions).  A stage covers 128 K columns, so every row
//    contributes one full 128-byte cache line per stage: fetching half
//    lines (64 K columns) halves the L2->LDS rate (27 vs 57 B/clk/CU
//    measured).
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
// Scaling (SCALE):
//  0  per-tensor fp32 scalars, applied in the epilogue (neutral E8M0
//     scales in the MFMA);
//  1  per-(row, K-block) power-of-two exponents (int8, [K/bs, rows], the
//     reference's block format).  An MFMA lane holds 32 consecutive K
//     values of one row, which lie in a single block for bs >= 32, so the
//     exponent goes straight into the MFMA's E8M0 scale operand (bias 127)
//     and the hardware applies it: no per-block partial sums or rescaling.
//     The MFMA reads its scale from byte 0 of the operand VGPR whatever the
//     opsel field says, so each sub-step has its own scale register.
//     The exponent -128 (the
//     reference's "zero W_lo block" sentinel, whose codes are all zero)
//     becomes the E8M0 code 0 (2^-127).
//
// The DMA is issued from inline assembly: the compiler's wait-count pass
// does not know these writes do not alias the LDS reads of the other
// buffer and would otherwise drain all loads before every LDS read.  Wait
// counts for the DMA are therefore explicit (s_waitcnt before the barrier).
//
// Stage layout (BM + 2*BN rows of 128 bytes): activation rows, then slot-0
// weight rows, then slot-1 weight rows.  The eight 16-byte chunks of a row
// are permuted by swz(row) = (row >> 1) & 7, which makes the MFMA operand
// reads (32 consecutive rows, same chunk) bank-conflict free on the
// 64-bank (256 B/clk) LDS.

typedef int v4i __attribute__((ext_vector_type(4)));
typedef uint32_t v2u __attribute__((ext_vector_type(2)));
#define TCFP_LDS __attribute__((address_space(3)))

constexpr int kSK = 128;                 // K columns per stage
constexpr int kRowB = kSK;               // bytes per stage row
constexpr uint32_t kOob = 0x80000000u;   // beyond every descriptor's range

TCFP_DEV int swz(int row) { return (row >> 1) & 7; }

// (the words are wave-uniform; readfirstlane states it for the compiler,
// whose uniformity analysis can lose track of it in kernels with divergent
// stores, and the DMA's inline assembly needs them in SGPRs)
TCFP_DEV v4i make_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  v4i r;
  r[0] = __builtin_amdgcn_readfirstlane(int(uint32_t(a)));
  r[1] = __builtin_amdgcn_readfirstlane(int(uint32_t(a >> 32) & 0xFFFFu));  // stride 0: raw bytes
  r[2] = __builtin_amdgcn_readfirstlane(int(bytes));  // num_records: bytes in range
  r[3] = 0x00020000;                                  // gfx9 raw-buffer data format word
  return r;
}

// 64 lanes x 16 bytes from rsrc + voff + soff into LDS [lds, lds + 1024).
TCFP_DEV void dma16(v4i rsrc, uint32_t voff, uint32_t soff, uint32_t lds) {
  asm volatile("buffer_load_dwordx4 %0, %1, %2 offen lds"
               :
               : "v"(voff), "s"(rsrc), "s"(soff), "{m0}"(lds)
               : "memory");
}

// dma16 with the non-temporal hint (data read once: kept out of the way of
// the operands in L2 and the Infinity Cache).
TCFP_DEV void dma16_nt(v4i rsrc, uint32_t voff, uint32_t soff, uint32_t lds) {
  asm volatile("buffer_load_dwordx4 %0, %1, %2 offen nt lds"
               :
               : "v"(voff), "s"(rsrc), "s"(soff), "{m0}"(lds)
               : "memory");
}

// 16 bytes from a per-lane global address into LDS at lds + 16 * lane
// (lds wave-uniform); counted by vmcnt like dma16.
TCFP_DEV void gdma16(const void* src, uint32_t lds) {
  asm volatile("global_load_lds_dwordx4 %0, off" : : "v"(src), "{m0}"(lds) : "memory");
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

// Unscaled FP8 MFMA (per-tensor scales are applied in the epilogue).  The
// compiler has no separate builtin for v_mfma_f32_32x32x64_f8f6f4: it selects
// that instruction for the scaled builtin when both scale operands are the
// literal 0, and the scaled form (an extra instruction word and two scale
// registers) otherwise.  The GEMM tests would see a scaled form with code 0
// (2^-127 per operand) at once: every product would vanish.
template <int BF, int AF>
TCFP_DEV v16f mfma_plain(const v8i& a, const v8i& b, const v16f& c) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, BF, AF, 0, 0, 0, 0);
}

// E8M0 code of a block exponent (bias 127; -128 and anything below -127
// map to code 0 = 2^-127).
TCFP_DEV uint32_t e8m0_of(int e) { return e < -127 ? 0u : uint32_t(e + 127); }

// Operand-format code for bf16 elements (the fp8 codes 0 = E4M3 and
// 1 = E5M2 double as the MFMA's cbsz / blgp format selectors).
constexpr int kBF16 = 16;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef int v4i_ __attribute__((ext_vector_type(4)));

// 16-byte half q of a 32-byte fragment as eight bf16.
TCFP_DEV bf16x8 bf16_half(const v8i& f, int q) {
  const v4i_ h = q == 0 ? v4i_{f[0], f[1], f[2], f[3]} : v4i_{f[4], f[5], f[6], f[7]};
  return __builtin_bit_cast(bf16x8, h);
}

// Pairs idx in [lo, hi) of a sub-step's (fragment, m-block) pairs (fragment
// idx % nf) that remain when the W_lo fragments (>= nb) are left out.
constexpr int pairs_in(int lo, int hi, int nf, int nb, bool with_lo) {
  int c = 0;
  for (int idx = lo; idx < hi; ++idx) c += (with_lo || idx % nf < nb) ? 1 : 0;
  return c;
}

struct GemmArgs {
  const uint8_t* A;
  const uint8_t* B0;
  const uint8_t* B1;
  int M, N, K;       // K and the leading dimensions count bytes of an
  int64_t lda, ldb;  // operand row: elements for fp8, 2 x elements for bf16
  const float* s_a;  // per-tensor scalars (SCALE 0), or fp32 block multipliers
  const float* s_0;  // (SCALE 2): [K/bs, M], [K/bs, N], [K/bs, N]
  const float* s_1;
  const int8_t* e_a;  // block exponents (SCALE 1): [K/bs, M], [K/bs, N], [K/bs, N]
  const int8_t* e_0;
  const int8_t* e_1;
  int bs_shift;  // log2(block size) (SCALE 1 and 2)
  const float* bias;
  void* out;
  int64_t ldo;
  int tiles_m, tiles_n;
  // split-K (SCALE 0 only): gridDim.y > 1 splits the contraction into
  // chunks of kc bytes; split y reads K columns [y*kc, y*kc + kc) and writes
  // its partial output at out + y*split_stride (fp32, no bias)
  int kc;
  int64_t split_stride;
  // (gemm_nt_dma_kernel) kwrap_b > 0: the B operand rows hold kwrap_b bytes
  // of contraction and byte k >= kwrap_b reads byte k - kwrap_b (K <= 2
  // kwrap_b, kwrap_b % 128 == 0): one copy serves a contraction that runs
  // over the same B columns twice
  int kwrap_b;
  // GELU epilogues of the persistent fp32 kernel (same leading dimension
  // ldo as out; EPI 2 ignores bias).  EPI 1 writes out (= h) as EPI 0 and the GELU amax rule's
  // keys of h (common.h) to part[2 * blockIdx.x], part[2 * blockIdx.x + 1].
  // EPI 2 reads the GELU derivative factors from aux and writes
  // aux * value (the GELU backward), with the workgroup's max |written
  // value| (float bits) at part[blockIdx.x] and, when cs_part is not null,
  // the 64-row column partials to cs_part ([M / 64, N]).
  const float* aux;
  uint32_t* part;
  float* cs_part;
  // In-kernel activation quantisation (gemm_nt_dma_kernel AQ != 0): A is the
  // bf16 / fp32 activation (lda in bytes); the tiles of output column 0
  // write its E4M3 codes to q_out ([M, K], row stride K) and its exponents
  // to e_out ([K/bs, M]) when q_out is not null.
  uint8_t* q_out;
  int8_t* e_out;
};

// NS = LDS stages in flight (2, or 4 for the small tile when one
// workgroup per CU is resident): the DMA of stage t + NS is issued once
// every wave has read stage t, so it has NS - 1 stages of MFMA time to land.
// F32BS (SCALE 2, and AQ): log2 of the block size, fixed per instantiation so
// that each block size compiles to one fold schedule (one segment reduction).
// AQ (SCALE 1 dual, 128 x 64 tile): 0 = A is FP8 codes with exponents e_a;
// 1 / 2 = A is the bf16 / fp32 activation, block-quantised to E4M3 inside
// the kernel (the reference's fused activation-quant GEMM).
template <int AF, int BF, bool SPLIT, typename OutT, int NW, int BM, int BN, int SCALE, int NS,
          int F32BS = 0, int AQ = 0>
__global__ __launch_bounds__(NW * 64, (NW == 4 && NS == 2 && BM <= 128 ? 2 : 1)) void gemm_nt_dma_kernel(
    GemmArgs g) {
  static_assert((SCALE == 2 || AQ != 0) == (F32BS != 0), "fp32 block scales and AQ fix the block size");
  // AQ: bf16 activations on the 128 x 64 tile; fp32 ones (twice the bytes
  // per stage in registers) on a 64 x 64 tile
  static_assert(AQ == 0 || (SCALE == 1 && !SPLIT && AF == 0 && NS == 2 && NW == 4 && BN == 64 &&
                            (BM == 64 || (BM == 128 && AQ == 1))),
                "in-kernel activation quantisation: E4M3 block-scaled dual GEMM, 128/64 x 64 tile");
  constexpr int f32_bsh = F32BS;
  constexpr int WM = NW / 2;        // wave rows
  constexpr int TMW = BM / WM;      // activation rows per wave
  constexpr int MB = TMW / 32;      // 32-row m-blocks per wave
  constexpr int TNW = BN / 2;       // weight rows per wave and slot
  constexpr int NB = TNW / 32;      // 32-row n-blocks per wave and slot
  constexpr int NF = 2 * NB;        // weight fragments per sub-step
  constexpr int SROWS = BM + 2 * BN;
  constexpr int STAGE = SROWS * kRowB;
  // stage rows DMA'd by each wave (with AQ the waves quantise the activation
  // rows themselves and DMA only the weight rows)
  constexpr int RPW = (AQ ? 2 * BN : SROWS) / NW;
  constexpr int DI = RPW / 8;       // 1 KiB DMA instructions per wave and stage
  static_assert(RPW % 16 == 0 && BM % RPW == 0 && BN % RPW == 0, "DMA rows must tile regions");
  static_assert(MB >= 1 && NB >= 1, "tile too small for the wave grid");
  static_assert(NS == 2 || (NS == 4 && SCALE == 0), "deep pipelines carry no exponent loads");
  static_assert(SCALE != 2 || (NW == 4 && BM == 128 && BN == 64 && NS == 2),
                "fp32 block scales use the 128 x 64 tile");
  // SCALE 2: a three-slot ring of per-stage fp32 scale areas (up to four
  // K-blocks of 1 KiB) behind the operand stages
  constexpr int kScB = SCALE == 2 ? 4096 : 0;
  // AQ: the activation exponents of the two buffered stages, [buffer][32-K
  // block of the stage][row] (a block of bs >= 32 columns fills
  // kSK / bs of the four slots)
  constexpr int kExB = AQ ? 2 * (kSK / 32) * BM : 0;
  // AQ: per-wave scratch of one float per (row, block) segment of a stage
  constexpr int kAqS = AQ ? NW * (BM / NW) * (kSK >> F32BS) * 4 : 0;
  __shared__ __align__(16) uint8_t lds[NS * STAGE + 3 * kScB + kExB + kAqS];

  const int M = g.M, N = g.N;
  int K = g.K;
  OutT* __restrict__ out = static_cast<OutT*>(g.out);
  int64_t koff = 0;  // byte offset of this split's first K column
  if constexpr (SCALE == 0) {
    if (gridDim.y > 1) {
      koff = int64_t(blockIdx.y) * g.kc;
      K = min(g.kc, g.K - int(koff));
      out += int64_t(blockIdx.y) * g.split_stride;
    }
  }

  // ---- tile mapping (XCD-aware, grouped) ----
  const int T = g.tiles_m * g.tiles_n;
  int l = blockIdx.x;
  if ((T & 7) == 0) l = (l & 7) * (T >> 3) + (l >> 3);
  // 4 tile-rows per group: the 32 workgroups an XCD runs at once share 4
  // A panels (8 wide groups re-read a large A once per 4 column tiles: the
  // 16384 x 4096 x 16384 split-bf16 wgrad ran 1.80 ms grouped by 8 against
  // 1.69 ms by 4; C3 and C4 shapes measured the same either way)
  constexpr int G = 4;
  const int per_group = G * g.tiles_n;
  const int first_m = (l / per_group) * G;
  const int gm = min(g.tiles_m - first_m, G);
  const int tm = first_m + (l % per_group) % gm;
  const int tn = (l % per_group) / gm;
  const int m0 = tm * BM;
  const int n0 = SPLIT ? tn * (2 * BN) : tn * BN;
  const int n1 = SPLIT ? n0 + BN : n0;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int lr = lane & 31, lg = lane >> 5;

  // ---- this wave's DMA source: its RPW stage rows lie in the activation,
  // slot-0 or slot-1 region
  const int srow0 = (AQ ? BM : 0) + wave * RPW;
  const uint8_t* src;
  int64_t ld;
  int rows_left, row_base;
  if (srow0 < BM) {
    src = g.A + koff + int64_t(m0) * g.lda; ld = g.lda; rows_left = min(M - m0, BM); row_base = srow0;
  } else if (srow0 < BM + BN) {
    src = g.B0 + (g.kwrap_b ? 0 : koff) + int64_t(n0) * g.ldb; ld = g.ldb;
    rows_left = min(N - n0, BN); row_base = srow0 - BM;
  } else {
    src = g.B1 + (g.kwrap_b ? 0 : koff) + int64_t(n1) * g.ldb; ld = g.ldb;
    rows_left = min(N - n1, BN); row_base = srow0 - BM - BN;
  }
  // a wrapping B region addresses contraction bytes koff + t * kSK modulo kwrap_b
  const uint32_t kwrap = srow0 >= BM ? uint32_t(g.kwrap_b) : 0u;
  const uint32_t nrec =
      rows_left > 0 ? uint32_t(int64_t(rows_left - 1) * ld + (kwrap ? int(kwrap) : K)) : 0u;
  const v4i rsrc = make_rsrc(src, nrec);
  // Instruction i fills stage rows srow0 + i*8 .. +8 (1 KiB); lane writes row
  // +lane/8 at physical chunk lane%8.  srow0 is a multiple of 16, so the
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

  // ---- fp32 block scales (SCALE 2).  Stage t's K-block b (of kSK / bs) is
  // brought into ring slot t % 3 by wave b with one 1 KiB global->LDS load:
  // lanes 0-31 carry the 128 activation-row multipliers, lanes 32-47 the 64
  // slot-0 and lanes 48-63 the 64 slot-1 weight-row multipliers, 4 floats
  // each.  Groups past the matrix re-read its last group (M, N % 4 == 0);
  // their rows are never stored.
  const float* sc_src = nullptr;
  int sc_ld = 0;
  if constexpr (SCALE == 2) {
    if (lane < 32) {
      sc_src = g.s_a + min(m0 + 4 * lane, M - 4);
      sc_ld = M;
    } else {
      const int nb = lane < 48 ? n0 : n1;
      sc_src = (lane < 48 ? g.s_0 : g.s_1) + min(nb + 4 * ((lane - 32) & 15), N - 4);
      sc_ld = N;
    }
  }
  const uint32_t sc_lds =
      uint32_t(reinterpret_cast<uintptr_t>((TCFP_LDS uint8_t*)lds)) + uint32_t(NS * STAGE);
  const int nkb = SCALE == 2 ? (K >> f32_bsh) : 0;

  // DMA of stage t (K columns t*128 ..) into buffer t & 1.  Stages past the
  // end are issued as all-out-of-range loads (zeros into a buffer nobody
  // reads again), so the issue stays branch-free.
  auto issue = [&](int t) {
    const uint32_t dst = lds_base + uint32_t(t & (NS - 1)) * STAGE;
    const bool live = t < nt;
    uint32_t soff = uint32_t(live ? t : 0) * kSK;
    if (kwrap) {
      soff += uint32_t(koff);
      if (soff >= kwrap) soff -= kwrap;
    }
    const bool last = t == nt - 1;
#pragma unroll
    for (int i = 0; i < DI; ++i) {
      const int c = (i & 1) ? chunk1 : chunk0;
      dma16(rsrc, (!live || (last && c * 16 >= krem)) ? kOob : voff[i], soff, dst + i * 1024);
    }
    if constexpr (SCALE == 2) {
      if (live && wave < (kSK >> f32_bsh)) {
        const int kb = min(((t * kSK) >> f32_bsh) + wave, nkb - 1);
        gdma16(sc_src + int64_t(kb) * sc_ld, sc_lds + uint32_t(t % 3) * kScB + uint32_t(wave) * 1024);
      }
    }
  };

  // ---- in-kernel activation quantisation (AQ).  A stage's BM x 128
  // activation tile is loaded into registers (16 bytes per lane and round,
  // ALPR lanes per row: consecutive lanes hold consecutive K columns, so a
  // (row, K-block) segment lies in AL adjacent lanes), block-quantised with
  // block_quant_kernel's rule -- max |x| over the segment, exponent
  // max(ceil(log2(amax / 448)), -126), codes RNE(clamp(x * 2^-e, 448)) --
  // and written as E4M3 codes into the stage's activation rows (swizzled as
  // the DMA would write them) and as exponents into the stage's exponent
  // slots.  The tiles of output column 0 also store the codes and
  // exponents to q_out / e_out.
  constexpr int AES = AQ == 2 ? 4 : 2;             // input element bytes
  constexpr int AVEC = 16 / AES;                    // elements per lane and round
  constexpr int ALPR = kSK / AVEC;                  // lanes per stage row
  constexpr int ARPI = 64 / ALPR;                   // rows per wave and round
  constexpr int ARL = AQ ? BM / (NW * ARPI) : 1;    // rounds per stage
  constexpr int AL = AQ ? (1 << f32_bsh) / AVEC : 1;  // lanes per (row, block) segment
  uint4 ar[ARL];
  const int arow = AQ ? wave * ARPI + lane / ALPR : 0;  // tile row of round 0
  const int acol = AQ ? (lane % ALPR) * AVEC : 0;       // column within the stage
  const int arows = min(M - m0, BM);
  const uint32_t anrec =
      (AQ && arows > 0) ? uint32_t(int64_t(arows - 1) * g.lda + int64_t(K) * AES) : 0u;
  const __amdgpu_buffer_rsrc_t arsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(g.A) + int64_t(m0) * g.lda, 0, int(anrec), 0x00020000);
  const uint32_t avoff0 = uint32_t(arow) * uint32_t(g.lda) + uint32_t(acol * AES);
  const uint32_t astride = uint32_t(NW * ARPI) * uint32_t(g.lda);  // bytes between rounds
  // loads of stage t's activation (rows past M and columns past K read 0)
  auto aload = [&](uint4* a4, int t) {
    if constexpr (AQ != 0) {
      const uint32_t soff = uint32_t(t) * (kSK * AES);
      const bool kin = t * kSK + acol < K;
#pragma unroll
      for (int r = 0; r < ARL; ++r) {
        const bool in = kin && arow + r * NW * ARPI < arows;
        a4[r] = __builtin_bit_cast(
            uint4, __builtin_amdgcn_raw_buffer_load_b128(arsrc, in ? avoff0 + r * astride : kOob,
                                                         soff, 0));
      }
    }
  };
  int8_t* const exs = reinterpret_cast<int8_t*>(lds + NS * STAGE + 3 * kScB);
  // side outputs through buffer stores: a store beyond the descriptor's
  // range is dropped, so rows past M and columns past K need no branches
  const bool side = AQ != 0 && g.q_out != nullptr && tn == 0;
  const uint32_t qnrec = side && arows > 0 ? uint32_t(int64_t(arows) * K) : 0u;
  const __amdgpu_buffer_rsrc_t qrsrc = __builtin_amdgcn_make_buffer_rsrc(
      g.q_out + int64_t(m0) * K, 0, int(qnrec), 0x00020000);
  const uint32_t enrec = side ? uint32_t(int64_t(K >> f32_bsh) * M) : 0u;
  const __amdgpu_buffer_rsrc_t ersrc =
      __builtin_amdgcn_make_buffer_rsrc(g.e_out, 0, int(enrec), 0x00020000);
  // A wave's stage holds ASEG (row, block) segments.  Their maxima go to
  // the wave's scratch slots; each lane then turns at most two of them into
  // an exponent (written to the MFMA's exponent slots and e_out) and a
  // multiplier 2^-e (written back over the maximum), which the segment's
  // lanes read for the conversion: one exponent evaluation per segment
  // instead of one per lane.
  constexpr int NSB = AQ ? kSK >> f32_bsh : 1;              // blocks per stage row
  constexpr int ASEG = AQ ? ARL * ARPI * NSB : 1;           // segments per wave and stage
  float* const aslot = reinterpret_cast<float*>(lds + NS * STAGE + 3 * kScB + kExB) + wave * ASEG;
  auto aquant = [&](const uint4* a4, int t) {
    if constexpr (AQ != 0) {
      uint8_t* st = lds + (t & 1) * STAGE;
      int8_t* ex = exs + (t & 1) * (kSK / 32) * BM;
      const int sb = acol >> f32_bsh;                        // block of this lane's columns
      // 1. segment maxima (|x| as bits: unsigned order, NaN above inf)
      uint32_t am[ARL];
#pragma unroll
      for (int r = 0; r < ARL; ++r) {
        const uint32_t w[4] = {a4[r].x, a4[r].y, a4[r].z, a4[r].w};
        uint32_t a;
        if constexpr (AQ == 2) {
          a = umax(umax(absbits(__uint_as_float(w[0])), absbits(__uint_as_float(w[1]))),
                   umax(absbits(__uint_as_float(w[2])), absbits(__uint_as_float(w[3]))));
        } else {
          // bf16 magnitudes, two per word: max of the 16-bit halves
          typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
          u16x2 m = __builtin_bit_cast(u16x2, w[0] & 0x7FFF7FFFu);
#pragma unroll
          for (int q = 1; q < 4; ++q)
            m = __builtin_elementwise_max(m, __builtin_bit_cast(u16x2, w[q] & 0x7FFF7FFFu));
          a = uint32_t(m[0] > m[1] ? m[0] : m[1]) << 16;
        }
        am[r] = seg_umax<AL>(a);
        aslot[(r * ARPI + lane / ALPR) * NSB + sb] = __uint_as_float(am[r]);
      }
      // 2. one exponent per segment (lanes past ASEG repeat a segment)
#pragma unroll
      for (int i = 0; i < (ASEG + 63) / 64; ++i) {
        const int sid = (lane + 64 * i) % ASEG;
        const int e = block_exponent(aslot[sid], kE4M3Max);
        aslot[sid] = exp2i(-e);
        const int wr = sid / NSB, b = sid % NSB;
        const int row = wave * ARPI + wr % ARPI + (wr / ARPI) * NW * ARPI;
        ex[b * BM + row] = int8_t(e);
        if (side) {
          const int gk = t * kSK + (b << f32_bsh);
          const uint32_t eoff = gk < K && row < arows
                                    ? uint32_t(gk >> f32_bsh) * uint32_t(M) + uint32_t(m0 + row)
                                    : kOob;
          __builtin_amdgcn_raw_buffer_store_b8(uint8_t(e), ersrc, eoff, 0, 0);
        }
      }
      // 3. codes
#pragma unroll
      for (int r = 0; r < ARL; ++r) {
        const int row = arow + r * NW * ARPI;
        const float mul = aslot[(r * ARPI + lane / ALPR) * NSB + sb];
        const uint32_t w[4] = {a4[r].x, a4[r].y, a4[r].z, a4[r].w};
        // |x| <= amax, so the clamp changes nothing unless amax * 2^-e
        // exceeds 448 (or is NaN) somewhere in the wave
        const bool clamp = __builtin_amdgcn_ballot_w64(!(__uint_as_float(am[r]) * mul <= kE4M3Max)) != 0;
        uint32_t c[AVEC / 4];
        if (AQ == 1 && !clamp) {
          // v_cvt_scalef32_pk_fp8_bf16 with a power-of-two scale 2^e is
          // RNE(x * 2^-e) for every in-range bf16 x (a GPU test runs every
          // finite bf16 at every exponent the rule yields against the
          // multiply-clamp-convert path); out of range it yields NaN, not
          // 448 -- waves holding such a block take the clamping branch
          typedef short v2s __attribute__((ext_vector_type(2)));
          typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
          // 2^e from 2^-e: both normal for every finite input (-126 <= e <= 120)
          const float sc = __uint_as_float(0x7F000000u - __float_as_uint(mul));
#pragma unroll
          for (int q = 0; q < AVEC / 4; ++q) {
            v2s r2 = {0, 0};
            r2 = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(r2, __builtin_bit_cast(v2bf, w[2 * q]), sc, false);
            r2 = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(r2, __builtin_bit_cast(v2bf, w[2 * q + 1]), sc, true);
            c[q] = __builtin_bit_cast(uint32_t, r2);
          }
        } else {
          float v[AVEC];
          if constexpr (AQ == 2) {
#pragma unroll
            for (int q = 0; q < 4; ++q) v[q] = __uint_as_float(w[q]);
          } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              v[2 * q] = __uint_as_float(w[q] << 16);
              v[2 * q + 1] = __uint_as_float(w[q] & 0xFFFF0000u);
            }
          }
#pragma unroll
          for (int q = 0; q < AVEC; ++q) v[q] = v[q] * mul;
          if (clamp) {
#pragma unroll
            for (int q = 0; q < AVEC; ++q) v[q] = clampf(v[q], kE4M3Max);
          }
#pragma unroll
          for (int q = 0; q < AVEC / 4; ++q)
            c[q] = cvt4_fp8<TCFP_FP8_E4M3>(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
        }
        const int off = row * kRowB + ((((acol >> 4) ^ swz(row))) << 4) + (acol & 15);
        const int gk = t * kSK + acol;
        const uint32_t qoff =
            gk < K && row < arows ? uint32_t(row) * uint32_t(K) + uint32_t(gk) : kOob;
        if constexpr (AQ == 2) {
          *reinterpret_cast<uint32_t*>(st + off) = c[0];
          if (side) __builtin_amdgcn_raw_buffer_store_b32(c[0], qrsrc, qoff, 0, 0);
        } else {
          *reinterpret_cast<uint2*>(st + off) = make_uint2(c[0], c[1]);
          if (side)
            __builtin_amdgcn_raw_buffer_store_b64(v2u{c[0], c[1]}, qrsrc, qoff, 0, 0);
        }
      }
    }
  };
  // activation exponents of stage t from the exponent slots, per
  // (m-block, sub-step) as load_raw lays them out
  auto aexps = [&](int* rw_, int t) {
    if constexpr (AQ != 0) {
      const int8_t* ex = exs + (t & 1) * (kSK / 32) * BM;
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < MB; ++i)
          rw_[2 * (NF + i) + h] = ex[((h * 64 + lg * 32) >> f32_bsh) * BM + wm * TMW + i * 32 + lr];
    }
  };

  // ---- per-lane LDS read offsets: sub-step h, 16-byte half q of a fragment.
  // The MFMA takes byte j of lane l as K index 16*(l/32) + 32*(j/16) + j%16
  // of its 64-wide step, and the E8M0 scale of lane l covers the 32-wide K
  // block l/32 -- i.e. bytes 16*(l/32) .. +15 of BOTH lane halves.  So lane
  // half g loads 16-byte chunks g and 2 + g of the sub-step: its scale then
  // covers exactly the 32 K columns 32*g .. 32*g + 31 that one block of the
  // exponent arrays describes.  (For unscaled products any K order works.)
  int ro[2][2];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int q = 0; q < 2; ++q) ro[h][q] = lr * kRowB + (((4 * h + lg + 2 * q) ^ swz(lr)) << 4);

  // ---- block exponents (SCALE 1).  Fragment q's weight row is
  // rw + dq(q) and fragment i's activation row is ra + 32*i; offsets into
  // the [K/bs, rows] exponent arrays are 32-bit from uniform bases.
  const uint32_t rw = uint32_t(n0 + wn * TNW + lr);
  const uint32_t ra = uint32_t(m0 + wm * TMW + lr);
  auto dq = [&](int q) { return uint32_t(((q / NB) ? n1 - n0 : 0) + (q % NB) * 32); };
  // Raw exponents of stage t, one register per (fragment, sub-step); rows
  // or K past the matrix read as 0 (2^0, multiplying zero operands).
  auto load_raw = [&](int* raw, int t) {
    if constexpr (SCALE == 1) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int k = t * kSK + h * 64 + lg * 32;
        const bool kin = k < K;
        const uint32_t kb = uint32_t(k >> g.bs_shift);
        const uint32_t ow = kb * uint32_t(N) + rw, oa = kb * uint32_t(M) + ra;
#pragma unroll
        for (int q = 0; q < NF; ++q) {
          const int8_t* e = (!SPLIT && (q / NB)) ? g.e_1 : g.e_0;
          raw[2 * q + h] = (kin && rw + dq(q) < uint32_t(N)) ? int(e[ow + dq(q)]) : 0;
        }
        if constexpr (AQ == 0) {
#pragma unroll
          for (int i = 0; i < MB; ++i)
            raw[2 * (NF + i) + h] =
                (kin && ra + 32 * i < uint32_t(M)) ? int(g.e_a[oa + 32 * i]) : 0;
        }
      }
    }
  };
  // E8M0 operand per (fragment, sub-step).  The scale always comes from
  // byte 0 of the VGPR (the MFMA's opsel does not select other bytes), so
  // each sub-step gets its own register.
  auto pack = [&](uint32_t* sc, const int* raw) {
    if constexpr (SCALE == 1) {
#pragma unroll
      for (int f = 0; f < 2 * (NF + MB); ++f) sc[f] = e8m0_of(raw[f]);
    }
  };

  // [slot][n-block][m-block].  Block-scaled dual GEMMs keep one set: with
  // exponents the MFMA applies each slot's scales, so W_hi and W_lo
  // products add directly; with fp32 scales each K-block's products are
  // folded into it on the VALU.
  constexpr int NACC = (SCALE != 0 && !SPLIT) ? 1 : 2;
  v16f acc[NACC][NB][MB];
#pragma unroll
  for (int s = 0; s < NACC; ++s)
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[s][j][i][r] = 0.0f;

  // Fragments of sub-step h of stage t: [0, NF) weights (slot, n-block),
  // [NF, NF + MB) activations (m-block).
  auto read_frags = [&](v8i* f, int t, int h) {
    const uint8_t* st = lds + (t & (NS - 1)) * STAGE;
#pragma unroll
    for (int q = 0; q < NF; ++q) {
      const int rb = (BM + (q / NB) * BN + wn * TNW + (q % NB) * 32) * kRowB;
      f[q] = make_frag(lds_read16(st, rb + ro[h][0]), lds_read16(st, rb + ro[h][1]));
    }
#pragma unroll
    for (int i = 0; i < MB; ++i) {
      const int rb = (wm * TMW + i * 32) * kRowB;
      f[NF + i] = make_frag(lds_read16(st, rb + ro[h][0]), lds_read16(st, rb + ro[h][1]));
    }
  };
  // W_lo sparsity (SCALE 1 dual): a stage whose W_lo exponents are the
  // -128 sentinel on every lane of the wave (E8M0 code 0; the quantisers
  // write all-zero codes there) contributes nothing, so its W_lo MFMAs are
  // skipped (tcfp/kernels.py:766-776 with the default threshold 0).
  constexpr bool kSkipLo = SCALE == 1 && !SPLIT;
  auto lo_live = [&](const uint32_t* scv) -> bool {
    if constexpr (kSkipLo) {
      uint32_t o = 0;
#pragma unroll
      for (int q = NB; q < NF; ++q) o |= scv[2 * q] | scv[2 * q + 1];
      return __builtin_amdgcn_ballot_w64(o != 0u) != 0;
    } else {
      return true;
    }
  };
  // One MFMA of weight fragment q and activation fragment i, sub-step h
  auto mfma1 = [&](const v8i* f, const uint32_t* scv, int h, int q, int i) {
    v16f& c = acc[(q / NB) % NACC][q % NB][i];
    if constexpr (AF == kBF16) {
      // a fragment holds 16 bf16 K values: two K=16 MFMAs
      c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bf16_half(f[q], 0), bf16_half(f[NF + i], 0),
                                                  c, 0, 0, 0);
      c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bf16_half(f[q], 1), bf16_half(f[NF + i], 1),
                                                  c, 0, 0, 0);
    } else if constexpr (SCALE == 1) {
      c = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
          f[q], f[NF + i], c, BF, AF, 0, int(scv[2 * q + h]), 0, int(scv[2 * (NF + i) + h]));
    } else {
      c = mfma_plain<BF, AF>(f[q], f[NF + i], c);
    }
  };
  // One sub-step (h) of MFMAs; `sc` holds the stage's E8M0 scales.  LO
  // false (a std::integral_constant) leaves out the W_lo fragments.
  auto mfmas = [&](const v8i* f, const uint32_t* scv, int h, auto lo) {
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int q = 0; q < NF; ++q) {
        if constexpr (kSkipLo && !decltype(lo)::value) {
          if (q >= NB) continue;
        }
        mfma1(f, scv, h, q, i);
      }
  };
  // MFMAs of (fragment, m-block) pairs [lo, hi) of sub-step h, pairs in
  // m-block-major order as in mfmas
  auto mfmas_range = [&](const v8i* f, const uint32_t* scv, int h, int lo, int hi, auto live) {
#pragma unroll
    for (int idx = 0; idx < NF * MB; ++idx) {
      if (idx < lo || idx >= hi) continue;
      const int i = idx / NF, q = idx % NF;
      if constexpr (kSkipLo && !decltype(live)::value) {
        if (q >= NB) continue;
      }
      mfma1(f, scv, h, q, i);
    }
  };
  // NF*MB MFMAs (NB*MB without W_lo) and 2*(NF+MB) LDS reads per sub-step:
  // spread the reads evenly
  auto interleave = [&](auto lo) {
    constexpr int nmf = (kSkipLo && !decltype(lo)::value) ? NB * MB : NF * MB;
    interleave_mfma_lds<nmf * (AF == kBF16 ? 2 : 1), 2 * (NF + MB), 0>();
  };
  // All DMA issued so far has landed and every wave's LDS reads are done
  // (gfx9 s_waitcnt: vmcnt bits [3:0] and [15:14], expcnt [6:4], lgkmcnt [11:8]).
  // sched_barrier(0) keeps the scheduler from moving MFMAs across it: MFMAs
  // touch no memory, so without it they drift past the barrier and the LDS
  // reads before it are left with nothing to hide behind.
  // With NS stages, the DMAs of stages t+2 .. t+NS-1 may stay in flight.
  constexpr int kInflight = (NS - 2) * DI;
  // four stages in flight on one four-wave workgroup per CU
  constexpr bool kDeep = NW == 4 && NS == 4 && SCALE == 0 && AQ == 0;
  auto sync_all = [&]() {
    __builtin_amdgcn_sched_barrier(0);
    // vmcnt(kInflight) lgkmcnt(0), expcnt untouched
    __builtin_amdgcn_s_waitcnt((kInflight & 15) | (7 << 4) | ((kInflight >> 4) << 14));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  };

  v8i f0[NF + MB], f1[NF + MB];
  uint32_t sc[2 * (NF + MB)];  // E8M0 scales of the current stage
  int raw[2 * (NF + MB)];   // exponents of the next stage, in flight
  if (nt > 0) {
    load_raw(raw, 0);
    if constexpr (AQ != 0) aload(ar, 0);
#pragma unroll
    for (int s = 0; s < NS; ++s) issue(s);
    if constexpr (AQ != 0) {
      // stage 0's activation into buffer 0 (waiting for its loads waits for
      // the DMAs issued after them too), then stage 1's loads; the barrier
      // waits for the LDS writes only
      aquant(ar, 0);
      if (nt > 1) aload(ar, 1);
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0), vmcnt and expcnt untouched
    } else {
      // wait for stage 0 only: the DMAs of stages 1 .. NS-1 may stay in flight
      // (the exponent loads were issued before all of them and are complete;
      // a wave that also loads fp32 scales issues one more per stage, which
      // only makes this wait longer)
      constexpr int kPro = (NS - 1) * DI;
      __builtin_amdgcn_s_waitcnt((kPro & 15) | (7 << 4) | ((kPro >> 4) << 14));
    }
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if constexpr (AQ != 0) aexps(raw, 0);
    pack(sc, raw);
    read_frags(f0, 0, 0);
    if constexpr (kDeep) read_frags(f1, 0, 1);
  }
  if constexpr (SCALE == 2) {
    // Per K-block partial products p (fresh accumulators), folded into acc
    // with the block's fp32 multipliers once the block's MFMAs are done:
    //   acc += s_a[m] * (s_0[n] * p_0 + s_1[n] * p_1)   (dual)
    //   acc_s += (s_s[n] * s_a[m]) * p_s                 (split single GEMM)
    // With 32-wide blocks each 64-wide MFMA is issued twice, once per lane
    // half: the other half's E8M0 scales are set to 2^-127 on both operands,
    // which scales its products by 2^-254, far below the smallest fp32
    // subnormal, so they round to zero.
    v16f p[2][NB][MB];
    const v16f zero16 = {};
    auto mfma_p = [&](const v8i* f, auto fresh, int sl) {
#pragma unroll
      for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int q = 0; q < NF; ++q) {
          v16f& c = p[q / NB][q % NB][i];
          if constexpr (decltype(fresh)::value)
            c = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(f[q], f[NF + i], zero16, BF, AF, 0,
                                                                 sl, 0, sl);
          else
            c = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(f[q], f[NF + i], c, BF, AF, 0, sl,
                                                                 0, sl);
        }
    };
    auto fold = [&](int t, int b) {
      const float* sb = reinterpret_cast<const float*>(lds + NS * STAGE + (t % 3) * kScB + b * 1024);
      float sa[MB];
#pragma unroll
      for (int i = 0; i < MB; ++i) sa[i] = sb[wm * TMW + i * 32 + lr];
      // lane holds n rows 8 * (r / 4) + 4 * lg + r % 4 of each 32-row block
#pragma unroll
      for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) {
          const int c = wn * TNW + j * 32 + 8 * gq + 4 * lg;
          const float4 u4 = *reinterpret_cast<const float4*>(sb + 128 + c);
          const float4 v4 = *reinterpret_cast<const float4*>(sb + 192 + c);
          const float w0[4] = {u4.x, u4.y, u4.z, u4.w}, w1[4] = {v4.x, v4.y, v4.z, v4.w};
#pragma unroll
          for (int i = 0; i < MB; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int r = 4 * gq + e;
              if constexpr (SPLIT) {
                acc[0][j][i][r] = __builtin_fmaf(p[0][j][i][r], w0[e] * sa[i], acc[0][j][i][r]);
                acc[1][j][i][r] = __builtin_fmaf(p[1][j][i][r], w1[e] * sa[i], acc[1][j][i][r]);
              } else {
                const float u = __builtin_fmaf(p[1][j][i][r], w1[e], p[0][j][i][r] * w0[e]);
                acc[0][j][i][r] = __builtin_fmaf(u, sa[i], acc[0][j][i][r]);
              }
            }
        }
    };
    constexpr int bsh = f32_bsh;
    auto substep = [&](const v8i* f, int t, int h) {
      if constexpr (bsh == 5) {
        mfma_p(f, std::true_type{}, lg == 0 ? 127 : 0);
        fold(t, 2 * h);
        mfma_p(f, std::true_type{}, lg == 1 ? 127 : 0);
        fold(t, 2 * h + 1);
      } else if constexpr (bsh == 6) {
        mfma_p(f, std::true_type{}, 127);
        fold(t, h);
      } else if (h == 0) {
        mfma_p(f, std::true_type{}, 127);
      } else {
        mfma_p(f, std::false_type{}, 127);
        fold(t, 0);
      }
    };
    for (int t = 0; t < nt; ++t) {
      read_frags(f1, t, 1);
      substep(f0, t, 0);
      // stage t + 1 and its scales landed, every wave has its stage-t
      // fragments and is past stage t - 1's scales: refill t's buffer and
      // ring slot (t + 2) % 3 == (t - 1) % 3
      sync_all();
      issue(t + NS);
      __builtin_amdgcn_sched_barrier(0);
      read_frags(f0, t + 1, 0);
      substep(f1, t, 1);
    }
  } else if constexpr (BM == 256 && NS == 2) {
    // Large tile, one workgroup per CU: its 8 waves meet at every barrier, so
    // the MFMA pipes drain there.  Half of sub-step 0's MFMAs (operands
    // already in registers) are held back until after the barrier, and the
    // refill DMA is issued behind them, so the pipes restart at once.
    constexpr int NP = NF * MB;
    constexpr int MPP = AF == kBF16 ? 2 : 1;  // MFMAs per (fragment, m-block) pair
    for (int t = 0; t < nt; ++t) {
      load_raw(raw, t + 1);
      __builtin_amdgcn_sched_barrier(0);
      // the stage's body with or without its W_lo MFMAs
      auto body = [&](auto lv) {
        constexpr bool L = decltype(lv)::value || !kSkipLo;
        read_frags(f1, t, 1);
        mfmas_range(f0, sc, 0, 0, NP / 2, lv);
        interleave_mfma_lds<pairs_in(0, NP / 2, NF, NB, L) * MPP, 2 * (NF + MB), 0>();
        sync_all();
        mfmas_range(f0, sc, 0, NP / 2, NP, lv);
        __builtin_amdgcn_sched_barrier(0);
        issue(t + NS);
        __builtin_amdgcn_sched_barrier(0);
        read_frags(f0, t + 1, 0);
        mfmas(f1, sc, 1, lv);
        interleave(lv);
      };
      // (no W_lo skip here: a second copy of this body takes the register
      // headroom of the 256-row tile and spills)
      body(std::true_type{});
      pack(sc, raw);
    }
  } else if constexpr (kDeep) {
    // One wave per SIMD: nothing else on the SIMD covers a gap in the wave's
    // own MFMA stream.  A stage's fragments (both sub-steps) are read into
    // registers during the stage before, so its MFMAs wait for nothing.  The
    // barrier sits behind the stage's first MFMA (the refill's offsets are
    // formed in its shadow); the refill DMA is spread over the next six
    // MFMAs and the next stage's reads over the next five, so the last reads
    // have two MFMAs to land before the stage ends.  (A/B at 4096 x 1024 x
    // 8192 E5M2 x E4M3: 40.4 -> 34.4 us, bit-identical; two MFMAs ahead of
    // the barrier, or reads in every slot, measured slower.)
    constexpr int NFR = NF + MB;  // fragments per sub-step
    constexpr int NP = NF * MB;   // (fragment, m-block) pairs per sub-step
    constexpr int SL = 2 * NP;    // MFMA pairs (slots) per stage
    constexpr int DSL = 6;        // slots after the barrier that carry the DMA
    constexpr int RSL = 5;        // slots after the barrier that carry the reads
    static_assert(1 + DSL <= SL && 1 + RSL < SL, "deep schedule slots");
    v8i g0[NFR], g1[NFR];
    // chunks past K in the last stage (per lane, even / odd DMA instruction)
    const bool tail0 = chunk0 * 16 >= krem, tail1 = chunk1 * 16 >= krem;
    // stage t on fragments c (sub-steps 0 / 1); stage t + 1's read into x
    auto stage = [&](v8i* c0, v8i* c1, v8i* x0, v8i* x1, int t) {
      auto mf = [&](int s) {
        const int h = s / NP, idx = s % NP;
        mfma1(h ? c1 : c0, sc, h, idx % NF, idx / NF);
      };
      // fragment r of stage t + 1 (sub-step r / NFR)
      auto rd = [&](int r) {
        const int h = r / NFR, x = r % NFR;
        const uint8_t* st = lds + ((t + 1) & (NS - 1)) * STAGE;
        const int rb = x < NF ? (BM + (x / NB) * BN + wn * TNW + (x % NB) * 32) * kRowB
                              : (wm * TMW + (x - NF) * 32) * kRowB;
        (h ? x1 : x0)[x] = make_frag(lds_read16(st, rb + ro[h][0]), lds_read16(st, rb + ro[h][1]));
      };
      mf(0);
      __builtin_amdgcn_sched_barrier(0);
      // the refill of stage t + NS into stage t's buffer, as issue() forms it
      const int tr = t + NS;
      const bool live = tr < nt, last = tr == nt - 1;
      uint32_t soff = uint32_t(live ? tr : 0) * kSK;
      if (kwrap) {
        soff += uint32_t(koff);
        if (soff >= kwrap) soff -= kwrap;
      }
      uint32_t dst = lds_base + uint32_t(tr & (NS - 1)) * STAGE;
      uint32_t vo[DI];
#pragma unroll
      for (int i = 0; i < DI; ++i) {
        vo[i] = (!live || (last && ((i & 1) ? tail1 : tail0))) ? kOob : voff[i];
        asm volatile("" : "+v"(vo[i]));  // formed here, not next to its DMA
      }
      asm volatile("" : "+s"(soff), "+s"(dst));
      // stage t + 1 landed, every wave holds stage t's fragments
      sync_all();
#pragma unroll
      for (int s = 1; s < SL; ++s) {
        mf(s);
        __builtin_amdgcn_sched_barrier(0);
        const int j = s - 1;
        if (j < DSL) {
#pragma unroll
          for (int i = j * DI / DSL; i < (j + 1) * DI / DSL; ++i)
            dma16(rsrc, vo[i], soff, dst + i * 1024);
        }
        if (j < RSL) {
#pragma unroll
          for (int r = j * 2 * NFR / RSL; r < (j + 1) * 2 * NFR / RSL; ++r) rd(r);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    // two stages per trip: the fragment sets swap roles
    for (int t = 0; t < nt; t += 2) {
      stage(f0, f1, g0, g1, t);
      if (t + 1 < nt) stage(g0, g1, f0, f1, t + 1);
    }
  } else {
  for (int t = 0; t < nt; ++t) {
    // exponents of stage t + 1 (SCALE 1, NS 2): this stage's vmcnt(0) covers them
    load_raw(raw, t + 1);
    __builtin_amdgcn_sched_barrier(0);
    // the stage's body with or without its W_lo MFMAs
    auto body = [&](auto lv) {
      // sub-step 0 of stage t; fragments of sub-step 1 stream in
      read_frags(f1, t, 1);
      mfmas(f0, sc, 0, lv);
      interleave(lv);
      // AQ: the activation of stage t + 1 (loaded during stage t - 1) is
      // quantised into buffer (t + 1) & 1, which every wave finished
      // reading at the previous barrier
      if constexpr (AQ != 0) {
        if (t + 1 < nt) aquant(ar, t + 1);
      }
      // stage t + 1 landed, every wave has its stage-t fragments: refill t's buffer
      sync_all();
      issue(t + NS);
      if constexpr (AQ != 0) {
        if (t + 2 < nt) aload(ar, t + 2);
        if (t + 1 < nt) aexps(raw, t + 1);
      }
      __builtin_amdgcn_sched_barrier(0);
      // sub-step 1 of stage t; fragments of stage t + 1 sub-step 0 stream in
      // (after the last stage they read a stale buffer and are never used)
      read_frags(f0, t + 1, 0);
      mfmas(f1, sc, 1, lv);
      interleave(lv);
    };
    // (with AQ the stage body is not duplicated: its quantising code is
    // large, and the narrow GEMMs it serves gain nothing from the skip)
    if (AQ != 0 || lo_live(sc)) body(std::true_type{});
    else body(std::false_type{});
    pack(sc, raw);
  }
  }

  // ---- epilogue -----------------------------------------------------------
  // A lane holds rows m, columns n..n+3 of each 32x32 block: storing that
  // directly writes 16 bytes into each of 32 rows per instruction.  Instead
  // each wave stages its TNW-column tile (per slot) through its own LDS
  // region and stores whole row segments of 16-byte chunks.
  constexpr int EB = int(sizeof(OutT));      // output element bytes
  constexpr int RB = TNW * EB;               // bytes of one staged tile row
  constexpr int CPR = RB / 16;               // 16-byte chunks per row
  constexpr int RPI = 64 / CPR;              // rows per store instruction
  static_assert(NW * TMW * RB <= NS * STAGE, "epilogue staging must fit the operand buffers");
  uint8_t* eps = lds + wave * (TMW * RB);    // this wave's staging region
  float c0s = 1.0f, c1s = 1.0f;
  if (SCALE == 0 && g.s_a) {
    const float sa = *g.s_a;
    c0s = sa * *g.s_0;
    c1s = SPLIT ? c0s : sa * *g.s_1;
  }
  const bool vec = (g.ldo % (16 / EB)) == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0;
  // every wave is done with the operand buffers before they are reused
  __builtin_amdgcn_s_waitcnt(0x0070);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
#pragma unroll
  for (int s = 0; s < (SPLIT ? 2 : 1); ++s) {
    const int nb = (s ? n1 : n0) + wn * TNW;  // first output column of this tile
    // the lane's bias columns, loaded once for all its rows (16-byte loads
    // where the four columns are in range; the pointer is 16-byte aligned).
    // Not with fp32 block scales, whose single-GEMM block-32 variant has no
    // registers to spare for them.
    constexpr bool kBiasHoist = SCALE != 2;
    float4 bq[kBiasHoist ? NB * 4 : 1];
    if (kBiasHoist && g.bias) {
#pragma unroll
      for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) {
          const int c = nb + j * 32 + gq * 8 + lg * 4;
          if (c + 3 < N) {
            bq[j * 4 + gq] = *reinterpret_cast<const float4*>(g.bias + c);
          } else {
            bq[j * 4 + gq] = make_float4(c < N ? g.bias[c] : 0.0f, c + 1 < N ? g.bias[c + 1] : 0.0f,
                                         c + 2 < N ? g.bias[c + 2] : 0.0f, 0.0f);
          }
        }
    }
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) {
          const int row = i * 32 + lr, col = j * 32 + gq * 8 + lg * 4;
          float v[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int r = gq * 4 + q;
            if constexpr (SPLIT) v[q] = acc[s][j][i][r] * c0s;
            else if constexpr (NACC == 1) v[q] = acc[0][j][i][r];
            else v[q] = acc[0][j][i][r] * c0s + acc[NACC - 1][j][i][r] * c1s;
          }
          if (g.bias) {
            if constexpr (kBiasHoist) {
              const float4 b4 = bq[j * 4 + gq];
              v[0] += b4.x;
              v[1] += b4.y;
              v[2] += b4.z;
              v[3] += b4.w;
            } else {
#pragma unroll
              for (int q = 0; q < 4; ++q) v[q] += nb + col + q < N ? g.bias[nb + col + q] : 0.0f;
            }
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
        OutT* o = out + int64_t(m) * g.ldo + n;
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

// ---------------------------------------------------------------------------
// Persistent large-tile dual GEMM: per-tensor scales, bf16 or fp32 output.
//
// One workgroup per CU runs tiles b, b + G, b + 2G, ... (G = gridDim.x) of
// the same grouped, XCD-aware tile order as gemm_nt_dma_kernel, as one
// stream of K stages, so a tile change costs neither a workgroup launch nor
// a cold pipeline:
//  - stage 0 of the next tile is loaded while the current tile's last stage
//    computes (it takes the buffer stage nt - 2 frees);
//  - the last stage's buffer is not refilled: the epilogue stages the bf16
//    output there (every wave finished reading it at that stage's barrier),
//    reads it back into registers, and the next tile's stage 1 is loaded
//    into it before the global stores are issued;
//  - the first barrier of the next tile waits for that stage but not for the
//    stores (loads and stores retire in issue order under vmcnt), so the
//    output drains to memory while the next tile computes.
// The per-stage schedule is the large tile's of gemm_nt_dma_kernel.
// Launched only for full tiles (M % 256 == 0, N % 128 == 0, K % 128 == 0,
// K > 128: two stages at least) and a 16-byte aligned output with
// ldo % 8 == 0: every wave then issues exactly NST store instructions per
// tile, which the vmcnt accounting above relies on, and no stage is partial.
//
// fp32 output (OutT = float) skips the LDS staging: each lane stores its
// accumulator rows as 16-byte vectors straight from registers (16 stores per
// wave and tile), and the freed last-stage buffer takes the next tile's
// stage 1 right at the last stage's barrier.
//
// SCALE 1: block exponents (E8M0 MFMA scale operands, one accumulator set
// for W_hi and W_lo).  A stage's exponents are DMA'd into an LDS area of
// their own with the stage's operands (two instructions of 16-byte chunks
// of the exponent rows), read by each lane right after the barrier that
// makes them valid, and turned into E8M0 codes at the end of the stage.
//
// SPL (single GEMM, 256 x 64 slots): the two weight slots are two adjacent
// 64-row blocks of one B (the launcher points B1 / e_1 64 rows past B0 /
// e_0), each with its own accumulator set, written to the two 64-column
// halves of a 256 x 128 output tile.  Block-scaled single GEMMs keep two
// accumulator sets, which the 256 x 128 slots' registers do not hold; the
// 256 x 64 slots' do.
template <int AF, int BF, typename OutT, int EPI = 0, int SCALE = 0, int ND = 8, int BNT = 128,
          bool SPL = false>
__global__ __launch_bounds__(BNT == 128 && ND == 4 ? 256 : 512, 1) void gemm_nt_persist_kernel(
    GemmArgs g) {
  constexpr bool F32OUT = std::is_same<OutT, float>::value;
  static_assert(EPI == 0 || F32OUT, "GELU epilogues write fp32");
  static_assert(SCALE == 0 || (SCALE == 1 && EPI == 0), "block exponents: plain epilogue only");
  static_assert(!SPL || (EPI == 0 && F32OUT), "single GEMM: fp32, plain epilogue");
  constexpr int NACC = (SCALE == 1 && !SPL) ? 1 : 2;
  constexpr int NSL = SPL ? 2 : 1;  // output column blocks per tile
  // ROLL (single GEMM, 256 x 128 slots: a 256 x 256 output tile): the two
  // accumulator sets take 128 registers, so the weight fragments are not
  // double-buffered: each is re-read for the next sub-step as soon as its
  // MFMAs are issued (four weight and two activation fragments per wave in
  // flight besides the current two activation fragments, 64 registers
  // instead of 96).
  constexpr bool ROLL = SPL && BNT == 128;
  // W4 (ND = 4 with 256 x 128 slots): four waves, one per SIMD, each
  // owning 128 activation rows x 64 weight rows of both slots
  constexpr bool W4 = BNT == 128 && ND == 4;
  constexpr int NW = W4 ? 4 : 8, BM = 256, BN = BNT, NS = 2;
  // BN = 64 (EPI 2 only): the GELU derivative factors of the tile (256 x 64
  // fp32, 64 KiB) are brought into LDS beside the two 48 KiB operand stages
  // in pieces during the tile's K stages, so the epilogue reads them from
  // LDS.  With the 256 x 128 tile (2 x 64 KiB of stages) there is no room
  // for its 128 KiB of factors, and loading them in the epilogue, every CU
  // at once, left the matrix cores idle: 8192 x 4096 x 1024 ran 120.9 us
  // against 74.4 us with the loads taken out (timing copy).
  constexpr bool DGL = BNT == 64 && EPI == 2;
  static_assert(BNT == 128 || (BNT == 64 && EPI == 2 && SCALE == 0 && F32OUT) || SPL,
                "the 256 x 64 tile serves the GELU backward epilogue and single GEMMs");
  static_assert(!ROLL || SCALE == 1, "the rolling schedule serves block-scaled single GEMMs");
  constexpr int WM = NW / 2, TMW = BM / WM, MB = TMW / 32;
  constexpr int TNW = BN / 2, NB = TNW / 32, NF = 2 * NB;
  constexpr int SROWS = BM + 2 * BN;
  constexpr int STAGE = SROWS * kRowB;
  // ND = waves that issue the operand DMA: all eight for the 256 x 128
  // tile; six of 64 rows each for the 256 x 64 tile (four for the
  // activation rows, one per weight slot), whose other two waves bring in
  // the GELU derivative factors.  (Four DMA waves with twice the rows each,
  // letting the other four waves' output stores drain past the barriers,
  // gained <= 1 us on standalone 8192 x 4096 x 1024 GEMMs but cost 7 us per
  // step of the fused MLP training step, measured in one process.)
  static_assert(BNT == 128 ? (ND == 8 || ND == 4) : ND == 6,
                "DMA waves: all of them; six for the 256 x 64 tile");
  static_assert(!W4 || (SCALE == 0 && EPI == 0 && !SPL && !F32OUT),
                "the four-wave tile serves per-tensor dual GEMMs with bf16 output");
  constexpr int RPW = SROWS / ND;
  constexpr int DI = RPW / 8;
  constexpr int NP = NF * MB;
  // (W4: two DMA instructions behind each of half a sub-step's MFMAs, one
  // fragment read behind each of the other half's)
  static_assert(!W4 || (DI == NP && NF + MB == NP / 2), "four-wave stage layout");
  constexpr int RB = TNW * 2;      // bytes of one staged bf16 tile row
  constexpr int CPR = RB / 16;     // 16-byte chunks per row
  constexpr int RPI = 64 / CPR;    // rows per store instruction
  // store instructions per wave and tile
  constexpr int NST = F32OUT ? NSL * MB * NB * 4 : TMW / RPI;
  static_assert(F32OUT || NW * TMW * RB <= STAGE, "epilogue staging must fit one operand buffer");
  // (a DMA wave holds at most two stages' DMA and one tile's stores in flight)
  static_assert(NST + 2 * (DI + (SCALE == 1 ? 1 : 0)) <= 63, "vmcnt immediate");
  // EPI 2's column partials: a wave's rows are one 64-row group, its two
  // m-blocks the group's halves
  static_assert(EPI != 2 || (TMW == kColGroup && MB == 2), "wave rows vs. column groups");
  // The tile's bias columns (block exponents): loaded at the top of stage
  // max(nt - 2, 0) by the first BN threads and stored here after that
  // stage's barrier (which waits for every earlier load), read by the
  // epilogue after the last stage's barrier.  Loaded in the epilogue
  // itself, each wait for the bias also waits for the next tile's DMA and
  // the stores before it: 8192 x 16384 x 4096 with block exponents ran
  // 1302 us that way against 1018 us.  The per-tensor epilogues keep the
  // direct loads: there the staging code measured 2-4% slower with fp32
  // output and ~1% slower at 4096^3 with bf16 output and no bias.
  constexpr bool kBiasLds = SCALE == 1;
  // one LDS array: the operand stages, then the bias columns (block
  // exponents), then the derivative factors (DGL)
  constexpr int kBiasB = kBiasLds ? NSL * BN * 4 : 0;
  constexpr int kDgB = DGL ? BM * BN * 4 : 0;
  // W4: 1 KiB that the refill DMA of a stage with nothing to load writes
  // (zeros from an out-of-range offset), so that its issue needs no branch
  constexpr int kDumB = W4 ? 1024 : 0;
  // SCALE 1: the block exponents of a stage, [K block of the stage][stage
  // row] (activation rows, then the two weight slots' rows), one area per
  // operand buffer, DMA'd with the stage (two 1 KiB instructions of
  // per-lane 16-byte chunks: up to four K blocks at bs 32).
  constexpr int kExpStage = SCALE == 1 ? 2048 : 0;
  static_assert(SCALE != 1 || 4 * SROWS <= kExpStage, "a stage's exponents fit their area");
  __shared__ __align__(16) uint8_t lds[NS * STAGE + kBiasB + kDgB + kDumB + 2 * kExpStage];
  float* const bias_s = reinterpret_cast<float*>(lds + NS * STAGE);
  const float* const dgl = reinterpret_cast<const float*>(lds + NS * STAGE + kBiasB);
  // GELU epilogues: EPI 1 the lane's int / uint maxima of the h bits (the
  // amax rule's keys), EPI 2 its max |value| bits (in amx)
  uint32_t amx = 0;
  int32_t kimax = INT32_MIN;

  const int M = g.M, N = g.N, K = g.K;
  OutT* __restrict__ out = static_cast<OutT*>(g.out);
  const int T = g.tiles_m * g.tiles_n;
  const int ntile = (T - int(blockIdx.x) + int(gridDim.x) - 1) / int(gridDim.x);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int lr = lane & 31, lg = lane >> 5;

  // this wave's DMA rows: activation (region 0), slot 0 (1) or slot 1 (2)
  const bool dma_wave = W4 || wave < ND;
  const int srow0 = (dma_wave ? wave : 0) * RPW;
  const int region = srow0 < BM ? 0 : (srow0 < BM + BN ? 1 : 2);
  const int row_base = region == 0 ? srow0 : (region == 1 ? srow0 - BM : srow0 - BM - BN);
  const uint8_t* const src_base = region == 0 ? g.A : (region == 1 ? g.B0 : g.B1);
  const int64_t ld = region == 0 ? g.lda : g.ldb;
  const int region_rows = region == 0 ? BM : BN;
  const uint32_t nrec = uint32_t(int64_t(region_rows - 1) * ld + K);  // full tiles only
  const int chunk0 = (lane & 7) ^ swz(lane >> 3);
  const int chunk1 = (lane & 7) ^ swz(8 + (lane >> 3));
  // byte offsets of this lane's row within a tile for even / odd DMA
  // instructions (tile-independent); instruction i adds i * 8 rows to the
  // lane offset.  (Not to the SGPR offset: DMA with SGPR offsets past 64 KiB
  // read the wrong rows on gfx950 -- measured, results wrong, no fault.)
  const uint32_t voff0 = uint32_t(int64_t(row_base + (lane >> 3)) * ld + chunk0 * 16);
  const uint32_t voff1 = uint32_t(int64_t(row_base + (lane >> 3)) * ld + chunk1 * 16);
  const uint32_t row8 = uint32_t(8 * ld);
  const uint32_t lds0 = uint32_t(reinterpret_cast<uintptr_t>((TCFP_LDS uint8_t*)lds));
  const uint32_t lds_base = lds0 + uint32_t(srow0) * kRowB;
  const int nt = K / kSK;

  // tile `it` of this workgroup -> (m0, n0)
  auto tile_of = [&](int it, int& m0, int& n0) {
    int l = int(blockIdx.x) + it * int(gridDim.x);
    if ((T & 7) == 0) l = (l & 7) * (T >> 3) + (l >> 3);
    // groups of 4 tile-rows, as in gemm_nt_dma_kernel (A/B on two boxes
    // against 8: 4096^3 95.4 -> 93.9 us, 8192 x 4096 x 1024 fp32 out
    // 71.2 -> 67.5 us, 8192 x 16384 x 4096 block 1018 -> 952 us; 8192 x
    // 4096 x 16384 block 820 -> 842 us)
    constexpr int G = 4;
    const int per_group = G * g.tiles_n;
    const int first_m = (l / per_group) * G;
    const int gm = min(g.tiles_m - first_m, G);
    m0 = (first_m + (l % per_group) % gm) * BM;
    n0 = ((l % per_group) / gm) * (NSL * BN);
  };
  auto src_of = [&](int m0, int n0) {
    return make_rsrc(src_base + int64_t(region == 0 ? m0 : n0) * ld, nrec);
  };
  // DMA of stage t of the tile whose operand rows `rs` describes into buffer b
  auto issue = [&](const v4i& rs, int t, int b) {
    if (!dma_wave) return;
    const uint32_t dst = lds_base + uint32_t(b) * STAGE;
    const uint32_t soff = uint32_t(t) * kSK;
    // (W4: the lane offsets laundered here too -- precomputed, its sixteen
    // instruction offsets were spilled, and each reload waited for every
    // DMA before it)
    uint32_t vb0 = voff0, vb1 = voff1;
    if constexpr (W4) asm volatile("" : "+v"(vb0), "+v"(vb1));
#pragma unroll
    for (int i = 0; i < DI; ++i)
      dma16(rs, ((i & 1) ? vb1 : vb0) + uint32_t(i) * row8, soff, dst + i * 1024);
  };
  // DGL: the current tile's derivative factors into LDS.  Piece p (1 KiB:
  // tile rows 4p .. 4p + 3, 16 lanes per row) lands at dgl + p KiB with
  // each row's 16-byte chunk c at chunk c ^ (row & 15), so the epilogue's
  // reads (32 rows, one chunk each) spread over every bank.  The waves that
  // issue no operand DMA (ND .. NW - 1) load them: they wait for memory
  // only at the tile's last barrier, so the pieces -- read from HBM -- have
  // the rest of the tile to land.  (Issued by the DMA waves, each stage's
  // barrier waited for that stage's pieces: no faster than the epilogue
  // loads.)  Wave ND + w issues pieces w, w + (NW - ND), ..., its k-th at
  // stage k % min(nt - 1, 2): all of them in the tile's first two stages.
  // Spread over every stage, the last pieces left about one stage before
  // the last barrier and every tile waited there for an HBM round trip
  // (8192 x 4096 x 1024: 120.7 us, 86.2 us with no factor loads at all).
  constexpr int NDG = NW - ND;  // factor-loading waves
  const uint32_t dg_lds0 = lds0 + uint32_t(NS * STAGE + kBiasB);
  const uint32_t ldo_b = uint32_t(g.ldo) * 4u;
  const int dg_np = (DGL && !dma_wave) ? (BM / 4 - (wave - ND) + NDG - 1) / (NDG > 0 ? NDG : 1) : 0;
  const uint32_t dg_nrec = uint32_t(int64_t(BM - 1) * g.ldo * 4 + BN * 4);
  auto issue_dg = [&](const v4i& rs, int t) {
    if constexpr (DGL) {
      const int span = nt - 1 < 2 ? nt - 1 : 2;  // nt >= 2
      if (t >= span) return;
      for (int k = t; k < dg_np; k += span) {
        const int p = (wave - ND) + NDG * k;
        const int row = 4 * p + (lane >> 4);
        const uint32_t vo = uint32_t(row) * ldo_b + uint32_t(((lane & 15) ^ (row & 15)) * 16);
        dma16_nt(rs, vo, 0u, dg_lds0 + uint32_t(p) * 1024u);  // (read once)
      }
    }
  };

  int ro[2][2];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int q = 0; q < 2; ++q) ro[h][q] = lr * kRowB + (((4 * h + lg + 2 * q) ^ swz(lr)) << 4);

  v16f acc[NACC][NB][MB];
  auto zero_acc = [&]() {
#pragma unroll
    for (int s = 0; s < NACC; ++s)
#pragma unroll
      for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int i = 0; i < MB; ++i)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[s][j][i][r] = 0.0f;
  };
  // output value r of accumulator block (j, i)
  auto accv = [&](int j, int i, int r, float c0, float c1) -> float {
    if constexpr (SCALE == 1) return acc[0][j][i][r];
    else return acc[0][j][i][r] * c0 + acc[NACC - 1][j][i][r] * c1;
  };

  // ---- block exponents (SCALE 1).  Weight fragment q takes the exponent of
  // weight row n0 + wn * TNW + 32 * (q % NB) + lr of e_0 (slot 0) or e_1
  // (slot 1), activation fragment i that of row m0 + wm * TMW + 32 * i + lr
  // of e_a; sub-step h of stage t covers K block t * (kSK >> bs) +
  // ((64 h + 32 lg) >> bs) for this lane's 32-column half lg.
  const int bsh = SCALE == 1 ? g.bs_shift : 0;
  const uint32_t kbs = uint32_t(kSK >> bsh);  // K blocks per stage
  // The exponent DMA: waves 0 and 1 each move 64 chunks of 16 bytes, chunk
  // c = 64 * wave + lane holding K block c / (SROWS / 16) of stage rows
  // 16 * (c % (SROWS / 16)) .. + 15; chunks past the stage's K blocks
  // re-read chunk 0 into the unused rest of the area.  Issued with the
  // stage's operand DMA, so they land two stages ahead as the operands do
  // (loaded per lane at the top of the stage before, the exponents' wait at
  // the barrier was exposed: the whole exponent handling measured 7-8% of
  // the block GEMM's time).
  constexpr int kCpk = SROWS / 16;
  const int ec = (wave & 1) * 64 + lane;  // (the issuing pair rotates with the stage)
  const bool ein = SCALE == 1 && uint32_t(ec / kCpk) < kbs;
  const int ekb = ein ? ec / kCpk : 0, er0 = ein ? (ec % kCpk) * 16 : 0;
  const int ereg = er0 < BM ? 0 : (er0 < BM + BN ? 1 : 2);
  const int erow = ereg == 0 ? er0 : (ereg == 1 ? er0 - BM : er0 - BM - BN);
  const int8_t* const ebase = ereg == 0 ? g.e_a : (ereg == 1 ? g.e_0 : g.e_1);
  const int64_t eld = ereg == 0 ? M : N;
  const uint32_t exp_lds0 = lds0 + uint32_t(NS * STAGE + kBiasB + kDgB + kDumB);
  auto issue_e = [&](int mt, int ntl, int t, int b) {
    if constexpr (SCALE == 1) {
      // waves 2 (t % (ND / 2)) and 2 (t % (ND / 2)) + 1 (all of them DMA waves)
      if ((wave >> 1) == t % (ND / 2)) {
        const int8_t* src =
            ebase + (int64_t(t) * kbs + ekb) * eld + (ereg == 0 ? mt : ntl) + erow;
        gdma16(src, exp_lds0 + uint32_t(b) * kExpStage + uint32_t(wave & 1) * 1024u);
      }
    }
  };
  uint32_t sc[SCALE == 1 ? 2 * (NF + MB) : 1];
  // The exponents of weight fragment q / activation fragment i of sub-step
  // h are bytes [K block (64 h + 32 lg) >> bs][row] of the stage's area;
  // their E8M0 codes go to sc[2 q + h] / sc[2 (NF + i) + h].  An int8
  // exponent byte u becomes (u ^ 128) - 1 saturated at 0: e = -128 .. 127
  // map to 0 (2^-127, the sentinel too), 0, 1, ..., 254.
  // raw exponent bytes of the stage whose exponents sit in area b, read
  // right after the barrier that makes them valid (an LDS round trip at the
  // end of the stage delayed the next stage's first MFMAs), and their E8M0
  // codes formed at the end of the stage
  uint32_t raw[SCALE == 1 ? 2 * (NF + MB) : 1];
  auto read_exps = [&](int b) {
    if constexpr (SCALE == 1) {
      const uint8_t* ea = lds + NS * STAGE + kBiasB + kDgB + kDumB + b * kExpStage;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int kb = (64 * h + 32 * lg) >> bsh;
#pragma unroll
        for (int q = 0; q < NF; ++q)
          raw[2 * q + h] = ea[kb * SROWS + BM + (q / NB) * BN + wn * TNW + (q % NB) * 32 + lr];
#pragma unroll
        for (int i = 0; i < MB; ++i) raw[2 * (NF + i) + h] = ea[kb * SROWS + wm * TMW + i * 32 + lr];
      }
    }
  };
  auto pack = [&]() {
    if constexpr (SCALE == 1) {
#pragma unroll
      for (int f = 0; f < 2 * (NF + MB); ++f)
        sc[f] = __builtin_elementwise_sub_sat(raw[f] ^ 128u, 1u);
    }
  };
  // fragment x of sub-step h from buffer b: weight fragment x (x < NF) or
  // activation fragment x - NF
  auto read_one = [&](v8i& f, int b, int h, int x) {
    const uint8_t* st = lds + b * STAGE;
    const int rb = x < NF ? (BM + (x / NB) * BN + wn * TNW + (x % NB) * 32) * kRowB
                          : (wm * TMW + (x - NF) * 32) * kRowB;
    f = make_frag(lds_read16(st, rb + ro[h][0]), lds_read16(st, rb + ro[h][1]));
  };
  auto read_frags = [&](v8i* f, int b, int h) {
#pragma unroll
    for (int x = 0; x < NF + MB; ++x) read_one(f[x], b, h, x);
  };
  // weight fragment q times activation fragment i of sub-step h
  auto mfma_one = [&](const v8i& fq, const v8i& fi, int h, int q, int i) {
    v16f& c = acc[(q / NB) % NACC][q % NB][i];
    if constexpr (SCALE == 1)
      c = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
          fq, fi, c, BF, AF, 0, int(sc[2 * q + h]), 0, int(sc[2 * (NF + i) + h]));
    else
      c = mfma_plain<BF, AF>(fq, fi, c);
  };
  auto mfmas_range = [&](const v8i* f, int h, int lo, int hi) {
#pragma unroll
    for (int idx = 0; idx < NP; ++idx) {
      if (idx < lo || idx >= hi) continue;
      const int i = idx / NF, q = idx % NF;
      mfma_one(f[q], f[NF + i], h, q, i);
    }
  };
  // ROLL: the MFMAs of weight fragment q with both activation fragments
  // fa[NF .. NF + MB), then the fragment's register takes (weight
  // fragment q of sub-step h_next from buffer b_next)
  auto mfma_roll = [&](v8i* fw, const v8i* fa, int h, int q, int b_next, int h_next) {
#pragma unroll
    for (int i = 0; i < MB; ++i) mfma_one(fw[q], fa[NF + i], h, q, i);
#pragma unroll
    for (int i = 0; i < MB; ++i) asm volatile("" : "+v"(acc[(q / NB) % NACC][q % NB][i]));
    __builtin_amdgcn_sched_barrier(0);
    if (b_next >= 0) read_one(fw[q], b_next, h_next, q);
    __builtin_amdgcn_sched_barrier(0);
  };
  // The MFMAs of (fragment, m-block) pairs [lo, hi) stay where they are:
  // an empty volatile asm that reads and writes their accumulators keeps
  // the compiler from sinking them past the branches that follow (the
  // barrier's wait count and the refill DMA depend on the stage), which
  // would leave the matrix cores idle at every barrier.
  auto pin_range = [&](int lo, int hi) {
#pragma unroll
    for (int idx = 0; idx < NP; ++idx) {
      if (idx < lo || idx >= hi) continue;
      const int i = idx / NF, q = idx % NF;
      asm volatile("" : "+v"(acc[(q / NB) % NACC][q % NB][i]));
    }
  };
  // every DMA landed except the newest `keep` vector-memory operations
  // (the previous tile's output stores), every wave's LDS reads are done.
  // A wave that issues no operand DMA waits for its LDS reads only, except
  // (DGL) at the tile's last barrier (`fin`), where its factor loads land.
  auto sync_keep = [&](auto keep, bool fin) {
    constexpr int k = decltype(keep)::value;
    __builtin_amdgcn_sched_barrier(0);
    if (dma_wave)
      __builtin_amdgcn_s_waitcnt((k & 15) | (7 << 4) | ((k >> 4) << 14));
    else if (DGL && fin)
      __builtin_amdgcn_s_waitcnt(0 | (7 << 4));  // vmcnt(0) lgkmcnt(0)
    else
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0), vmcnt and expcnt untouched
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  };

  float c0s = 1.0f, c1s = 1.0f;
  if (SCALE == 0 && g.s_a) {
    const float sa = *g.s_a;
    c0s = sa * *g.s_0;
    c1s = sa * *g.s_1;
  }

  int m0, n0;
  tile_of(0, m0, n0);
  v4i cur = src_of(m0, n0);
  v8i f0[NF + MB], f1[NF + MB];
  zero_acc();
  // prologue: stages 0 and 1 of the first tile (nt >= 2 for this kernel),
  // after stage 0's exponents (complete at the wait, which leaves only the
  // newest DI operations in flight)
  issue_e(m0, n0, 0, 0);
  issue(cur, 0, 0);
  issue_e(m0, n0, 1, 1);
  issue(cur, 1, 1);
  __builtin_amdgcn_s_waitcnt((DI & 15) | (7 << 4) | ((DI >> 4) << 14));
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  read_exps(0);
  pack();
  read_frags(f0, 0, 0);

  int cb0 = 0;  // buffer of the current tile's stage 0
  for (int it = 0; it < ntile; ++it) {
    const bool more = it + 1 < ntile;
    v4i dgr{};
    if constexpr (DGL) dgr = make_rsrc(g.aux + int64_t(m0) * g.ldo + n0, dg_nrec);
    v4i nxt = cur;
    int m1 = 0, n1 = 0;
    if (more) {
      tile_of(it + 1, m1, n1);
      nxt = src_of(m1, n1);
    }
    for (int t = 0; t < nt; ++t) {
      const int b = (cb0 + t) & 1;
      __builtin_amdgcn_sched_barrier(0);
      const bool bias_stage =
          kBiasLds && g.bias != nullptr && t == (nt > 2 ? nt - 2 : 0) && tid < NSL * BN;
      float bv = 0.0f;
      if (bias_stage) bv = g.bias[n0 + tid];
      if constexpr (W4) {
        // One wave per SIMD: nothing else hides a stall, so the stage is
        // one fixed sequence.  Sub-step 0's first half with the fragments
        // of sub-step 1 read behind its MFMAs (RDP per MFMA); the barrier;
        // the refill DMA behind the next MFMAs (DMP instructions per MFMA),
        // the fragments of sub-step 0 of stage t + 1 behind the MFMAs after
        // it (one per MFMA; after the last stage: the next tile's stage 0,
        // stale after the last tile).  A stage with nothing to load (the
        // last: its buffer stages the output) still issues the refill
        // instructions, re-reading stage 0 of the tile into a dummy KiB, so
        // that the issue needs no branch.
        constexpr int RDP = 2, DMP = 1;
        // The refill's parameters -- the next tile's stage 0 when t + 2 ==
        // nt (nxt == cur when there is none: the dummy then re-reads the
        // current tile's stage 0) -- are formed behind the first MFMA whose
        // slot carries no reads: formed at the top of the stage, their ~30
        // scalar instructions delayed its first MFMA.  (The lane offsets
        // are laundered per stage, so that the sixteen instruction offsets
        // are formed one add each instead of being kept in sixteen
        // registers across the kernel.)
        v4i drs;
        uint32_t dsoff = 0, dbase = 0, dstep = 0, vb0 = 0, vb1 = 0;
        auto dma_params = [&]() {
          const bool in_tile = t + 2 < nt;
          const bool live = t + 2 < nt + int(more);
          drs = in_tile ? cur : nxt;
          dsoff = in_tile ? uint32_t(t + 2) * kSK : 0u;
          dbase = live ? lds_base + uint32_t(b) * STAGE : lds0 + uint32_t(NS * STAGE + kBiasB + kDgB);
          dstep = live ? 1024u : 0u;
          vb0 = voff0;
          vb1 = voff1;
          asm volatile("" : "+v"(vb0), "+v"(vb1));
        };
        constexpr int JP = (NF + MB + RDP - 1) / RDP;  // the first pre-barrier slot without reads
        static_assert(JP < NP / 2, "a pre-barrier slot for the refill parameters");
        // after pre-barrier MFMA j: sub-step 1 fragments j * RDP .. + RDP
        auto pre_op = [&](int j) {
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int u = 0; u < RDP; ++u)
            if (j * RDP + u < NF + MB) read_one(f1[j * RDP + u], b, 1, j * RDP + u);
          if (j == JP) dma_params();
          __builtin_amdgcn_sched_barrier(0);
        };
        // after post-barrier MFMA j: refill instructions j * DMP .. + DMP,
        // then (j >= DI / DMP) fragment j - DI / DMP of stage t + 1
        auto post_op = [&](int j) {
          __builtin_amdgcn_sched_barrier(0);
          if (j < DI / DMP) {
#pragma unroll
            for (int u = 0; u < DMP; ++u) {
              const int i = j * DMP + u;
              dma16(drs, ((i & 1) ? vb1 : vb0) + uint32_t(i) * row8, dsoff,
                    dbase + uint32_t(i) * dstep);
            }
          } else if (j - DI / DMP < NF + MB) {
            read_one(f0[j - DI / DMP], b ^ 1, 0, j - DI / DMP);
          }
          __builtin_amdgcn_sched_barrier(0);
        };
        static_assert(NF + MB <= RDP * (NP / 2), "sub-step 1's fragments within sub-step 0's first half");
        static_assert(DI / DMP + NF + MB <= NP + NP / 2, "refill and reads within the stage");
#pragma unroll
        for (int idx = 0; idx < NP / 2; ++idx) {
          mfma_one(f0[idx % NF], f0[NF + idx / NF], 0, idx % NF, idx / NF);
          pre_op(idx);
        }
#pragma unroll
        for (int idx = 0; idx < NP / 2; ++idx)
          asm volatile("" : "+a"(acc[(idx % NF / NB) % NACC][idx % NF % NB][idx / NF]));
        if (t == 0 && it > 0)
          sync_keep(std::integral_constant<int, NST>{}, false);
        else
          sync_keep(std::integral_constant<int, 0>{}, false);
#pragma unroll
        for (int idx = NP / 2; idx < NP; ++idx) {
          mfma_one(f0[idx % NF], f0[NF + idx / NF], 0, idx % NF, idx / NF);
          post_op(idx - NP / 2);
        }
#pragma unroll
        for (int idx = 0; idx < NP; ++idx) {
          mfma_one(f1[idx % NF], f1[NF + idx / NF], 1, idx % NF, idx / NF);
          post_op(NP / 2 + idx);
        }
        continue;
      }
      if constexpr (ROLL) {
        // sub-step 1's activation fragments, then sub-step 0 weight fragment
        // by weight fragment, each register re-read for sub-step 1 behind
        // its MFMAs.  All of sub-step 1's MFMAs follow the barrier (PRE = 0;
        // with one or two of its weight fragments before the barrier the
        // 4096^3 single block-64 GEMM ran 66.5 / 68.5 us against 63.8 us).
#pragma unroll
        for (int i = 0; i < MB; ++i) read_one(f1[NF + i], b, 1, NF + i);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int q = 0; q < NF; ++q) mfma_roll(f0, f0, 0, q, b, 1);
        constexpr int PRE = 0;  // sub-step 1 weight fragments before the barrier
#pragma unroll
        for (int q = 0; q < PRE; ++q) mfma_roll(f0, f1, 1, q, -1, 0);
        if (t == 0 && it > 0)
          sync_keep(std::integral_constant<int, NST>{}, false);
        else
          sync_keep(std::integral_constant<int, 0>{}, false);
        if (bias_stage) bias_s[tid] = bv;
        read_exps(b ^ 1);
        // the next weight fragment's MFMAs refill the pipes after the
        // barrier, then the refill DMA and sub-step 0 of stage t + 1 (after
        // the last stage: the next tile's stage 0, landed at this barrier;
        // stale and unused after the last tile) into the free registers
        mfma_roll(f0, f1, 1, PRE, -1, 0);
        if (t + 2 < nt) {
          issue_e(m0, n0, t + 2, b);
          issue(cur, t + 2, b);
        } else if (t + 2 == nt && more) {
          issue_e(m1, n1, 0, b);
          issue(nxt, 0, b);
        } else if (more) {
          issue_e(m1, n1, 1, b);
          issue(nxt, 1, b);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < MB; ++i) read_one(f0[NF + i], b ^ 1, 0, NF + i);
#pragma unroll
        for (int q = 0; q <= PRE; ++q) read_one(f0[q], b ^ 1, 0, q);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int q = PRE + 1; q < NF; ++q) mfma_roll(f0, f1, 1, q, b ^ 1, 0);
        pack();
        continue;
      }
      read_frags(f1, b, 1);
      mfmas_range(f0, 0, 0, NP / 2);
      interleave_mfma_lds<NP / 2, 2 * (NF + MB), 0>();
      pin_range(0, NP / 2);
      if (t == 0 && it > 0)
        sync_keep(std::integral_constant<int, NST>{}, t + 1 == nt);
      else
        sync_keep(std::integral_constant<int, 0>{}, t + 1 == nt);
      if (bias_stage) bias_s[tid] = bv;
      read_exps(b ^ 1);
      mfmas_range(f0, 0, NP / 2, NP);
      pin_range(NP / 2, NP);
      __builtin_amdgcn_sched_barrier(0);
      if (t + 2 < nt) {
        issue_e(m0, n0, t + 2, b);
        issue(cur, t + 2, b);
      } else if (t + 2 == nt && more) {
        issue_e(m1, n1, 0, b);
        issue(nxt, 0, b);  // the next tile's stage 0
      } else if (F32OUT && more) {
        issue_e(m1, n1, 1, b);
        issue(nxt, 1, b);  // the next tile's stage 1 (no output staging)
      }
      issue_dg(dgr, t);
      __builtin_amdgcn_sched_barrier(0);
      // sub-step 0 of stage t + 1 (after the last stage: the next tile's
      // stage 0, landed at this barrier; stale and unused after the last
      // tile).  EPI 2 reads it after the epilogue, whose loads need the
      // registers.
      if (EPI != 2 || t + 1 < nt) read_frags(f0, b ^ 1, 0);
      mfmas_range(f1, 1, 0, NP);
      interleave_mfma_lds<NP, 2 * (NF + MB), 0>();
      pack();  // the next stage's E8M0 codes (its sub-step 1 MFMAs are issued)
    }

    const int sb = (cb0 + nt - 1) & 1;
    const int nb = n0 + wn * TNW;
    if constexpr (F32OUT) {
      // ---- epilogue: 16-byte stores from the accumulators --------------------
      // (the next tile's stage 1 exponents first: the stores follow)
      if constexpr (EPI == 2) {
        // g = value * gelu'(h) factor.  Every factor load of the tile is
        // issued before any store: a wait for a load also waits for every
        // vector-memory operation issued before it (the next tile's stage 1,
        // issued at the last stage, has a head start).
        float4 dv[MB * NB * 4];
#pragma unroll
        for (int i = 0; i < MB; ++i)
#pragma unroll
          for (int j = 0; j < NB; ++j)
#pragma unroll
            for (int gq = 0; gq < 4; ++gq) {
              if constexpr (DGL) {
                const int row = wm * TMW + i * 32 + lr;
                const int c = (wn * TNW + j * 32 + gq * 8 + lg * 4) >> 2;
                dv[(i * NB + j) * 4 + gq] =
                    *reinterpret_cast<const float4*>(dgl + row * BN + ((c ^ (row & 15)) << 2));
              } else {
                const int64_t o = int64_t(m0 + wm * TMW + i * 32 + lr) * g.ldo + nb + j * 32 +
                                  gq * 8 + lg * 4;
                dv[(i * NB + j) * 4 + gq] = *reinterpret_cast<const float4*>(g.aux + o);
              }
            }
        // g replaces the first accumulator set in place (the registers of
        // the second set and of the factors free up as they are consumed)
#pragma unroll
        for (int i = 0; i < MB; ++i)
#pragma unroll
          for (int j = 0; j < NB; ++j)
#pragma unroll
            for (int gq = 0; gq < 4; ++gq) {
              const int col = j * 32 + gq * 8 + lg * 4;
              const int64_t o = int64_t(m0 + wm * TMW + i * 32 + lr) * g.ldo + nb + col;
              const float4 d = dv[(i * NB + j) * 4 + gq];
              float v[4];  // (a dgrad: no bias)
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                const int r = gq * 4 + q;
                v[q] = accv(j, i, r, c0s, c1s);
              }
              v[0] = v[0] * d.x;
              v[1] = v[1] * d.y;
              v[2] = v[2] * d.z;
              v[3] = v[3] * d.w;
              store4<float>(reinterpret_cast<float*>(out) + o, v[0], v[1], v[2], v[3]);
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                amx = umax(amx, absbits(v[q]));
                acc[0][j][i][gq * 4 + q] = v[q];
              }
            }
        if (g.cs_part) {
          // ys[j * 16 + gq * 4 + q]: g(row lr) + g(row 32 + lr) of the lane's
          // column j * 32 + gq * 8 + lg * 4 + q (the wave's 64-row group)
          float ys[NB * 16];
#pragma unroll
          for (int j = 0; j < NB; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) ys[j * 16 + r] = acc[0][j][0][r] + acc[0][j][1][r];
          // halving folds over the 32 row lanes (lane bits 4 ... 0): each
          // step keeps half of the columns and adds the partner lane's
          // values of them (row distances 16 ... 1, as kColGroup's order
          // sums them); with NB = 2 lane lr ends with the group sum of
          // column lr, with NB = 1 (16 columns per lane half) the last step
          // adds the partner's value of the same column and lanes lr, lr ^ 1
          // both hold it
#pragma unroll
          for (int d = 16, len = NB * 16; d >= 1; d >>= 1, len >>= 1) {
            const bool up = (lr & d) != 0;
            if (len >= 2) {
#pragma unroll
              for (int k = 0; k < len / 2; ++k) {
                const float give = up ? ys[k] : ys[k + len / 2];
                const float keep = up ? ys[k + len / 2] : ys[k];
                ys[k] = keep + __shfl_xor(give, d);
              }
            } else {
              ys[0] = ys[0] + __shfl_xor(ys[0], d);
            }
          }
          const int col = NB == 2 ? (lr >> 4) * 32 + ((lr >> 2) & 3) * 8 + lg * 4 + (lr & 3)
                                  : ((lr >> 3) & 3) * 8 + lg * 4 + ((lr >> 1) & 3);
          if (NB == 2 || (lr & 1) == 0)
            g.cs_part[int64_t((m0 + wm * TMW) / kColGroup) * N + nb + col] = ys[0];
        }
        // the next tile's first fragments (its stage 0 landed at the last
        // stage's barrier; stale and unused after the last tile)
        read_frags(f0, sb ^ 1, 0);
      } else {
        // (SPL: output column block sl of the tile from accumulator set sl)
#pragma unroll
        for (int sl = 0; sl < NSL; ++sl)
#pragma unroll
        for (int i = 0; i < MB; ++i)
#pragma unroll
          for (int j = 0; j < NB; ++j)
#pragma unroll
            for (int gq = 0; gq < 4; ++gq) {
              const int row = i * 32 + lr, col = sl * BN + j * 32 + gq * 8 + lg * 4;
              const int64_t o = int64_t(m0 + wm * TMW + row) * g.ldo + nb + col;
              float v[4];
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                const int r = gq * 4 + q;
                if constexpr (SPL)
                  v[q] = SCALE == 1 ? acc[sl][j][i][r] : acc[sl][j][i][r] * c0s;
                else
                  v[q] = accv(j, i, r, c0s, c1s);
              }
              if (g.bias) {
                if constexpr (kBiasLds) {
                  const float4 b4 = *reinterpret_cast<const float4*>(bias_s + wn * TNW + col);
                  v[0] += b4.x;
                  v[1] += b4.y;
                  v[2] += b4.z;
                  v[3] += b4.w;
                } else {
#pragma unroll
                  for (int q = 0; q < 4; ++q) v[q] += g.bias[nb + col + q];
                }
              }
              store4<float>(reinterpret_cast<float*>(out) + o, v[0], v[1], v[2], v[3]);
              if constexpr (EPI == 1) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                  const uint32_t b = __float_as_uint(v[q]);
                  kimax = max(kimax, int32_t(b));
                  amx = umax(amx, b);
                }
              }
            }
      }
      __builtin_amdgcn_sched_barrier(0);
      zero_acc();
      cb0 = sb ^ 1;
      cur = nxt;
        m0 = m1;
      n0 = n1;
      continue;
    }
    // ---- epilogue: stage through the last stage's buffer -------------------
    // (the lane index is laundered here, so the compiler derives the
    // epilogue's lane-dependent offsets after the K loop instead of keeping
    // them live across it, where no register is free for them)
    int lane_e = lane;
    asm volatile("" : "+v"(lane_e));
    const int lr_e = lane_e & 31, lg_e = lane_e >> 5;
    uint8_t* eps = lds + sb * STAGE + wave * (TMW * RB);
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) {
          const int row = i * 32 + lr_e, col = j * 32 + gq * 8 + lg_e * 4;
          float v[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int r = gq * 4 + q;
            v[q] = accv(j, i, r, c0s, c1s);
          }
          if (g.bias) {
            if constexpr (kBiasLds) {
              const float4 b4 = *reinterpret_cast<const float4*>(bias_s + wn * TNW + col);
              v[0] += b4.x;
              v[1] += b4.y;
              v[2] += b4.z;
              v[3] += b4.w;
            } else {
#pragma unroll
              for (int q = 0; q < 4; ++q) v[q] += g.bias[nb + col + q];
            }
          }
          const int byte = col * 2;
          const int chunk = (byte >> 4) ^ (row & (CPR - 1));
          store4<uint16_t>(reinterpret_cast<uint16_t*>(eps + row * RB + chunk * 16 + (byte & 15)),
                           v[0], v[1], v[2], v[3]);
        }
    asm volatile("" ::: "memory");
    // the NST staged chunks of this lane, held in named registers (an array
    // here is kept in scratch memory across the barrier below)
    static_assert(F32OUT || NST == 8 || NST == 16, "eight or sixteen store chunks per lane");
    auto staged = [&](int s) {
      const int row = s * RPI + lane_e / CPR, cl = lane_e % CPR;
      return *reinterpret_cast<const uint4*>(eps + row * RB + ((cl ^ (row & (CPR - 1))) * 16));
    };
    const uint4 d0 = staged(0), d1 = staged(1), d2 = staged(2), d3 = staged(3);
    const uint4 d4 = staged(4), d5 = staged(5), d6 = staged(6), d7 = staged(7);
    uint4 d8{}, d9{}, d10{}, d11{}, d12{}, d13{}, d14{}, d15{};
    if constexpr (NST == 16) {
      d8 = staged(8), d9 = staged(9), d10 = staged(10), d11 = staged(11);
      d12 = staged(12), d13 = staged(13), d14 = staged(14), d15 = staged(15);
    }
    if (more) {
      // every wave holds its staged output: the buffer takes the next tile's stage 1
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0), vmcnt and expcnt untouched
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      issue_e(m1, n1, 1, sb);
      issue(nxt, 1, sb);
    }
    __builtin_amdgcn_sched_barrier(0);
    auto put = [&](int s, const uint4& d) {
      const int row = s * RPI + lane_e / CPR, cl = lane_e % CPR;
      OutT* o = out + int64_t(m0 + wm * TMW + row) * g.ldo + nb + cl * 8;
      *reinterpret_cast<uint4*>(o) = d;
    };
    put(0, d0); put(1, d1); put(2, d2); put(3, d3);
    put(4, d4); put(5, d5); put(6, d6); put(7, d7);
    if constexpr (NST == 16) {
      put(8, d8); put(9, d9); put(10, d10); put(11, d11);
      put(12, d12); put(13, d13); put(14, d14); put(15, d15);
    }
    __builtin_amdgcn_sched_barrier(0);
    zero_acc();
    cb0 = sb ^ 1;  // the next tile's stage 0 sits in the other buffer
    cur = nxt;
    m0 = m1;
    n0 = n1;
  }
  if constexpr (EPI != 0) {
    // the workgroup's partials (no DMA is in flight after the last tile; the
    // barrier retires every wave's last LDS reads before the operand
    // buffer takes the per-wave maxima)
    uint32_t* const wmax = reinterpret_cast<uint32_t*>(lds);
    __syncthreads();
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
      amx = umax(amx, uint32_t(__shfl_xor(int(amx), d)));
      if constexpr (EPI == 1) kimax = max(kimax, __shfl_xor(kimax, d));
    }
    if (lane == 0) {
      wmax[wave] = amx;
      wmax[NW + wave] = uint32_t(kimax);
    }
    __syncthreads();
    if (tid == 0) {
      uint32_t m = wmax[0];
      int32_t k = int32_t(wmax[NW]);
#pragma unroll
      for (int w = 1; w < NW; ++w) {
        m = umax(m, wmax[w]);
        k = max(k, int32_t(wmax[NW + w]));
      }
      if constexpr (EPI == 1) {
        g.part[2 * blockIdx.x] = uint32_t(k);
        g.part[2 * blockIdx.x + 1] = m;
      } else {
        g.part[blockIdx.x] = m;
      }
    }
  }
}

// Largest byte span any DMA descriptor may cover (offsets are 32-bit and
// the out-of-range sentinel must stay beyond every span).
constexpr int64_t kMaxSpan = (int64_t(1) << 31) - (int64_t(1) << 20);

// Tile policy: 0 = automatic (block-scaled single GEMMs may take 256 x 256
// tiles; per-tensor dual GEMMs with bf16 output and K >= 8192 the
// four-wave persistent tile), 1 = always 256 x 128, 2 = always 128 x 64,
// 3 = 128 x 64 with eight waves in the one-round deep-pipeline case,
// 4 = 256 x 128 with one workgroup per tile (no persistent launch),
// 5 = the four-wave persistent 256 x 128 tile (per-tensor dual, bf16 out).
int g_tile_policy = 0;

int num_cus() {
  static int n = 0;
  if (n == 0) {
    int dev = 0, v = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
        v > 0)
      n = v;
    else
      n = 256;
  }
  return n;
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// The persistent large-tile launch: full 256 x 128 tiles, two K stages at
// least, more tiles than CUs, no split-K, and every DMA span within the
// descriptors' reach (tile policies 0 and 1 only).  fp8 dual GEMMs with
// per-tensor scales or block exponents, fp32 or bf16 output.
bool persist_eligible(const GemmArgs& ga) {
  if (g_tile_policy != 0 && g_tile_policy != 1 && g_tile_policy != 5) return false;
  if (ga.M % 256 != 0 || ga.N % 128 != 0 || ga.K % kSK != 0 || ga.K <= kSK) return false;
  if (ga.kc > 0 && ga.kc < ga.K) return false;
  if (ga.ldo % 8 != 0 || !al16(ga.out)) return false;
  if (int64_t(256) * ga.lda + ga.K >= kMaxSpan || int64_t(128) * ga.ldb + ga.K >= kMaxSpan)
    return false;
  return int64_t(ga.M / 256) * (ga.N / 128) > num_cus();
}

// The persistent kernel DMAs each stage's block exponents into LDS as
// 16-byte chunks of the exponent arrays: their bases must be 16-byte aligned
// (rows and columns of its full tiles are multiples of 64).
bool exps_al16(const GemmArgs& ga) {
  return al16(ga.e_a) && al16(ga.e_0) && (ga.e_1 == nullptr || al16(ga.e_1));
}

template <int AF, int BF, bool SPLIT, typename OutT, int SCALE>
int launch_gemm(GemmArgs ga, hipStream_t st) {
  const int m = ga.M, n = ga.N, k = ga.K;
  if constexpr (SCALE == 1 && SPLIT && AF != kBF16 && std::is_same<OutT, float>::value) {
    // block-scaled single GEMM with more full 256 x 128 tiles than CUs: the
    // persistent kernel with the two weight slots on adjacent weight-row
    // blocks (32-bit exponent offsets) -- 128-row slots (256 x 256 output
    // tiles) when there are at least as many of those as CUs (automatic
    // tile policy), else 64-row slots (256 x 128 output tiles)
    if (persist_eligible(ga) && exps_al16(ga) &&
        int64_t(k >> ga.bs_shift) * (m > n ? m : n) < int64_t(INT32_MAX)) {
      if (ga.bias != nullptr && (reinterpret_cast<uintptr_t>(ga.bias) & 15) != 0)
        return TCFP_ERR_ALIGN;
      GemmArgs gp = ga;
      if (g_tile_policy == 0 && n % 256 == 0 && int64_t(m / 256) * (n / 256) >= num_cus()) {
        gp.B1 = ga.B0 + 128 * ga.ldb;
        gp.e_1 = ga.e_0 + 128;
        gp.tiles_m = m / 256;
        gp.tiles_n = n / 256;
        gemm_nt_persist_kernel<AF, BF, float, 0, 1, 8, 128, true>
            <<<unsigned(num_cus()), 512, 0, st>>>(gp);
        return hipGetLastError() == hipSuccess ? TCFP_OK : TCFP_ERR_HIP;
      }
      gp.B1 = ga.B0 + 64 * ga.ldb;
      gp.e_1 = ga.e_0 + 64;
      gp.tiles_m = m / 256;
      gp.tiles_n = n / 128;
      gemm_nt_persist_kernel<AF, BF, float, 0, 1, 6, 64, true>
          <<<unsigned(num_cus()), 512, 0, st>>>(gp);
      return hipGetLastError() == hipSuccess ? TCFP_OK : TCFP_ERR_HIP;
    }
  }
  // large tile unless it would leave CUs idle
  const int big_tiles = ((m + 255) / 256) * ((n + (SPLIT ? 255 : 127)) / (SPLIT ? 256 : 128));
  // (block-scaled single GEMMs keep two accumulator sets, which only the
  // small tile fits in registers)
  const bool small = (SCALE == 1 && SPLIT) || SCALE == 2 || g_tile_policy == 2 || g_tile_policy == 3 ||
                     (g_tile_policy == 0 && big_tiles < num_cus());
  const int BMv = small ? 128 : 256, BNv = small ? 64 : 128;
  ga.tiles_m = (m + BMv - 1) / BMv;
  ga.tiles_n = (n + (SPLIT ? 2 * BNv : BNv) - 1) / (SPLIT ? 2 * BNv : BNv);
  if (ga.bias != nullptr && (reinterpret_cast<uintptr_t>(ga.bias) & 15) != 0) return TCFP_ERR_ALIGN;
  // 512 threads per workgroup at most; the tile index is an int in the kernel
  if (!grid_x_fits(int64_t(ga.tiles_m) * ga.tiles_n, 512)) return TCFP_ERR_SHAPE;
  const bool dma_ok = int64_t(BMv) * ga.lda + k < kMaxSpan && int64_t(BNv) * ga.ldb + k < kMaxSpan;
  if (dma_ok) {
    // split-K (SCALE 0): gridDim.y = number of K chunks
    const unsigned splits =
        (SCALE == 0 && ga.kc > 0 && ga.kc < k) ? unsigned((k + ga.kc - 1) / ga.kc) : 1u;
    const dim3 grid(unsigned(ga.tiles_m) * unsigned(ga.tiles_n), splits);
    // a small-tile launch that fits in one round gets the 4-stage pipeline
    // (one workgroup per CU, 128 KiB of LDS)
    const bool deep = SCALE == 0 && small && int64_t(grid.x) * splits <= num_cus();
    if (small && deep) {
      if constexpr (SCALE == 0) {
        // (the eight-wave tuning policy serves FP8 operands; bf16 takes the
        // four-wave tile under every policy)
        if (AF != kBF16 && g_tile_policy == 3) {
          if constexpr (AF != kBF16)
            gemm_nt_dma_kernel<AF, BF, SPLIT, OutT, 8, 128, 64, SCALE, 4><<<grid, 512, 0, st>>>(ga);
        } else
          gemm_nt_dma_kernel<AF, BF, SPLIT, OutT, 4, 128, 64, SCALE, 4><<<grid, 256, 0, st>>>(ga);
      }
    } else if (small) {
      if constexpr (SCALE == 2) {
        if (ga.bs_shift == 5)
          gemm_nt_dma_kernel<AF, BF, SPLIT, OutT, 4, 128, 64, SCALE, 2, 5><<<grid, 256, 0, st>>>(ga);
        else if (ga.bs_shift == 6)
          gemm_nt_dma_kernel<AF, BF, SPLIT, OutT, 4, 128, 64, SCALE, 2, 6><<<grid, 256, 0, st>>>(ga);
        else
          gemm_nt_dma_kernel<AF, BF, SPLIT, OutT, 4, 128, 64, SCALE, 2, 7><<<grid, 256, 0, st>>>(ga);
      } else {
        gemm_nt_dma_kernel<AF, BF, SPLIT, OutT, 4, 128, 64, SCALE, 2><<<grid, 256, 0, st>>>(ga);
      }
    } else if constexpr (!(SCALE == 1 && SPLIT) && SCALE != 2) {
      // more tiles than CUs, all of them full: one persistent workgroup
      // per CU runs its tiles back to back
      bool persist = false;
      if constexpr (!SPLIT && AF != kBF16) {
        // (block exponents: 32-bit exponent offsets)
        persist = persist_eligible(ga) &&
                  (SCALE == 0 || (exps_al16(ga) && int64_t(ga.K >> ga.bs_shift) *
                                                           (ga.M > ga.N ? ga.M : ga.N) <
                                                       int64_t(INT32_MAX)));
        if (persist) {
          if constexpr (SCALE == 0 && std::is_same<OutT, uint16_t>::value) {
            // the four-wave tile (one wave per SIMD, 128 x 64 x 2 per wave):
            // a K loop ~5% shorter in shader cycles at a ~2% lower clock
            // (power cap) and a longer per-tile epilogue, so it is taken
            // where the K loop dominates (measured: 4096^2 x 8192 185.7 vs
            // 187.8 us, x 16384 352.8 vs 370.3 us; 4096^3 level)
            if (g_tile_policy == 5 || (g_tile_policy == 0 && ga.K >= 8192)) {
              gemm_nt_persist_kernel<AF, BF, OutT, 0, 0, 4><<<unsigned(num_cus()), 256, 0, st>>>(ga);
              return hipGetLastError() == hipSuccess ? TCFP_OK : TCFP_ERR_HIP;
            }
          }
          gemm_nt_persist_kernel<AF, BF, OutT, 0, SCALE><<<unsigned(num_cus()), 512, 0, st>>>(ga);
        }
      }
      if (!persist)
        gemm_nt_dma_kernel<AF, BF, SPLIT, OutT, 8, 256, 128, SCALE, 2><<<grid, 512, 0, st>>>(ga);
    }
    return hipGetLastError() == hipSuccess ? TCFP_OK : TCFP_ERR_HIP;
  }
  // Operand panels whose byte span (BM rows of the leading dimension) reaches
  // 2 GiB do not fit the DMA descriptors' 32-bit offsets: K-contiguous
  // operands with K < ~8M always fit.
  return TCFP_ERR_SHAPE;
}

template <bool SPLIT, typename OutT, int SCALE>
int dispatch_fmt(int a_fmt, int b_fmt, const GemmArgs& ga, hipStream_t st) {
  if (a_fmt == TCFP_FP8_E4M3 && b_fmt == TCFP_FP8_E4M3) return launch_gemm<0, 0, SPLIT, OutT, SCALE>(ga, st);
  if (a_fmt == TCFP_FP8_E5M2 && b_fmt == TCFP_FP8_E4M3) return launch_gemm<1, 0, SPLIT, OutT, SCALE>(ga, st);
  if (a_fmt == TCFP_FP8_E4M3 && b_fmt == TCFP_FP8_E5M2) return launch_gemm<0, 1, SPLIT, OutT, SCALE>(ga, st);
  if (a_fmt == TCFP_FP8_E5M2 && b_fmt == TCFP_FP8_E5M2) return launch_gemm<1, 1, SPLIT, OutT, SCALE>(ga, st);
  return TCFP_ERR_DTYPE;
}

template <int SCALE>
int dispatch_all(int a_fmt, int b_fmt, bool dual, int out_dtype, const GemmArgs& ga,
                 hipStream_t st) {
  if (dual) {
    if (out_dtype == TCFP_DTYPE_F32) return dispatch_fmt<false, float, SCALE>(a_fmt, b_fmt, ga, st);
    return dispatch_fmt<false, uint16_t, SCALE>(a_fmt, b_fmt, ga, st);
  }
  if (out_dtype == TCFP_DTYPE_F32) return dispatch_fmt<true, float, SCALE>(a_fmt, b_fmt, ga, st);
  return dispatch_fmt<true, uint16_t, SCALE>(a_fmt, b_fmt, ga, st);
}

int check_common(int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldb, int64_t ldo,
                 const void* a, const void* b_hi, const void* b_lo, int out_dtype) {
  if (m < 0 || n < 0 || k < 0 || m > INT32_MAX || n > INT32_MAX || k > INT32_MAX)
    return TCFP_ERR_SHAPE;
  if (k % 16 != 0) return TCFP_ERR_SHAPE;
  if (lda < k || ldb < k || ldo < n) return TCFP_ERR_SHAPE;
  if (lda % 16 != 0 || ldb % 16 != 0) return TCFP_ERR_ALIGN;
  if (!al16(a) || !al16(b_hi) || (b_lo && !al16(b_lo))) return TCFP_ERR_ALIGN;
  if (out_dtype != TCFP_DTYPE_F32 && out_dtype != TCFP_DTYPE_BF16) return TCFP_ERR_DTYPE;
  return TCFP_OK;
}

}  // namespace

extern "C" int tcfp_dual_gemm(const uint8_t* a, int a_fmt, int64_t lda, const uint8_t* b_hi,
                              const uint8_t* b_lo, int b_fmt, int64_t ldb, int64_t m, int64_t n,
                              int64_t k, const float* s_a, const float* s_hi, const float* s_lo,
                              const float* bias, void* out, int out_dtype, int64_t ldo,
                              void* stream) {
  const int rc = check_common(m, n, k, lda, ldb, ldo, a, b_hi, b_lo, out_dtype);
  if (rc != TCFP_OK) return rc;
  if (!s_a || !s_hi || (b_lo && !s_lo)) return TCFP_ERR_SHAPE;
  if (m == 0 || n == 0) return TCFP_OK;
  GemmArgs ga{};
  ga.A = a; ga.B0 = b_hi; ga.B1 = b_lo ? b_lo : b_hi;
  ga.M = int(m); ga.N = int(n); ga.K = int(k); ga.lda = lda; ga.ldb = ldb;
  ga.s_a = s_a; ga.s_0 = s_hi; ga.s_1 = b_lo ? s_lo : s_hi;
  ga.bias = bias; ga.out = out; ga.ldo = ldo;
  return dispatch_all<0>(a_fmt, b_fmt, b_lo != nullptr, out_dtype, ga,
                         static_cast<hipStream_t>(stream));
}

namespace {

// One GELU-epilogue persistent launch (EPI 1 or 2) for fp8 operand formats.
// One GELU-epilogue persistent launch for the formats the fused MLP passes:
// EPI 1 (layer 1's forward) E4M3 activations, EPI 2 (layer 2's dgrad) E5M2
// gradients, E4M3 weights (other formats take the unfused path).  EPI 2
// runs the 256 x 64 tile with its derivative factors in LDS when `narrow`
// (tiles_n counts 64-column tiles then), else the 256 x 128 tile.
template <int EPI>
int launch_persist_gelu(const GemmArgs& ga, bool narrow, hipStream_t st) {
  const unsigned grid = unsigned(num_cus());
  constexpr int AF = EPI == 1 ? TCFP_FP8_E4M3 : TCFP_FP8_E5M2;
  bool done = false;
  if constexpr (EPI == 2) {
    if (narrow) {
      gemm_nt_persist_kernel<AF, 0, float, EPI, 0, 6, 64><<<grid, 512, 0, st>>>(ga);
      done = true;
    }
  }
  if (!done) gemm_nt_persist_kernel<AF, 0, float, EPI><<<grid, 512, 0, st>>>(ga);
  return hipGetLastError() == hipSuccess ? TCFP_OK : TCFP_ERR_HIP;
}

// The EPI 2 launch on the 256 x 64 tile: full tiles, more of them than CUs,
// and every operand, output and factor span within a descriptor's reach;
// contractions up to 2048 only.  Its main loop issues half the MFMAs per
// barrier of the 256 x 128 tile's: measured in one process (bit-identical
// results, call incl. the quantising pass), 8192 x 4096 x 1024 160.5 against
// 163.8 us, 8192 x 4096 x 4096 357.4 against 310.2 us.
bool dgelu_narrow_eligible(const GemmArgs& ga) {
  if (g_tile_policy != 0) return false;
  if (ga.M % 256 != 0 || ga.N % 64 != 0 || ga.K % kSK != 0 || ga.K <= kSK || ga.K > 2048)
    return false;
  if (ga.ldo % 8 != 0 || !al16(ga.out) || !al16(ga.aux)) return false;
  if (int64_t(256) * ga.lda + ga.K >= kMaxSpan || int64_t(64) * ga.ldb + ga.K >= kMaxSpan ||
      int64_t(255) * ga.ldo * 4 + 256 >= kMaxSpan)
    return false;
  return int64_t(ga.M / 256) * (ga.N / 64) > num_cus();
}

bool fp8_fmt_ok(int f) { return f == TCFP_FP8_E4M3 || f == TCFP_FP8_E5M2; }

}  // namespace

extern "C" int tcfp_dual_gemm_gelu_quantize(const uint8_t* a, int a_fmt, int64_t lda,
                                            const uint8_t* b_hi, const uint8_t* b_lo, int b_fmt,
                                            int64_t ldb, int64_t m, int64_t n, int64_t k,
                                            const float* s_a, const float* s_hi,
                                            const float* s_lo, const float* bias, float* h,
                                            float* act, float* dgelu, int fp8_fmt, uint8_t* q,
                                            uint8_t* q_t, float* inv_out, void* workspace,
                                            void* stream) {
  const int rc = check_common(m, n, k, lda, ldb, n, a, b_hi, b_lo, TCFP_DTYPE_F32);
  if (rc != TCFP_OK) return rc;
  if (!s_a || !s_hi || (b_lo && !s_lo)) return TCFP_ERR_SHAPE;
  if (!fp8_fmt_ok(fp8_fmt)) return TCFP_ERR_DTYPE;
  if (!workspace) return TCFP_ERR_WORKSPACE;
  if (!h || !al16(h) || (act && !al16(act)) || (dgelu && !al16(dgelu)) || !inv_out)
    return TCFP_ERR_ALIGN;
  if (bias && !al16(bias)) return TCFP_ERR_ALIGN;
  GemmArgs ga{};
  ga.A = a; ga.B0 = b_hi; ga.B1 = b_lo;
  ga.M = int(m); ga.N = int(n); ga.K = int(k); ga.lda = lda; ga.ldb = ldb;
  ga.s_a = s_a; ga.s_0 = s_hi; ga.s_1 = s_lo;
  ga.bias = bias; ga.out = h; ga.ldo = n;
  // the keys go to the workspace's second partial array (the first takes
  // the amax partials the quantising pass reads)
  uint32_t* keys = static_cast<uint32_t*>(workspace) + tcfp::max_parts();
  ga.part = keys;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (b_lo && a_fmt == TCFP_FP8_E4M3 && b_fmt == TCFP_FP8_E4M3 && m > 0 &&
      persist_eligible(ga) && 2 * num_cus() <= tcfp::max_parts()) {
    ga.tiles_m = int(m / 256);
    ga.tiles_n = int(n / 128);
    const int r = launch_persist_gelu<1>(ga, false, st);
    if (r != TCFP_OK) return r;
    return tcfp::gelu_quantize_from_keys(h, m, n, fp8_fmt, act, dgelu, q, q_t, inv_out,
                                         workspace, keys, num_cus(), stream);
  }
  // any other shape: the GEMM, then the GELU amax pass
  const int r = tcfp_dual_gemm(a, a_fmt, lda, b_hi, b_lo, b_fmt, ldb, m, n, k, s_a, s_hi, s_lo,
                               bias, h, TCFP_DTYPE_F32, n, stream);
  if (r != TCFP_OK) return r;
  return tcfp_gelu_quantize_per_tensor(h, m, n, fp8_fmt, act, dgelu, q, q_t, inv_out, workspace,
                                       stream);
}

extern "C" int tcfp_dual_gemm_dgelu_quantize_colsum(
    const uint8_t* a, int a_fmt, int64_t lda, const uint8_t* b_hi, const uint8_t* b_lo, int b_fmt,
    int64_t ldb, int64_t m, int64_t n, int64_t k, const float* s_a, const float* s_hi,
    const float* s_lo, const float* dgelu, float* grad, int fp8_fmt, uint8_t* q, uint8_t* q_t,
    float* inv_out, float* col_sum, void* workspace, void* colsum_ws, size_t colsum_ws_bytes,
    void* stream) {
  const int rc = check_common(m, n, k, lda, ldb, n, a, b_hi, b_lo, TCFP_DTYPE_F32);
  if (rc != TCFP_OK) return rc;
  if (!s_a || !s_hi || (b_lo && !s_lo)) return TCFP_ERR_SHAPE;
  if (!fp8_fmt_ok(fp8_fmt)) return TCFP_ERR_DTYPE;
  if (n % 8 != 0) return TCFP_ERR_SHAPE;
  if (!workspace) return TCFP_ERR_WORKSPACE;
  if (!dgelu || !grad || !al16(dgelu) || !al16(grad) || !inv_out) return TCFP_ERR_ALIGN;
  const bool sums = col_sum != nullptr && m > 0 && n > 0;
  if (sums && (!colsum_ws || colsum_ws_bytes < tcfp_colsum_workspace_bytes(m, n)))
    return TCFP_ERR_WORKSPACE;
  if (sums && (!al16(colsum_ws) || !al16(col_sum))) return TCFP_ERR_ALIGN;
  GemmArgs ga{};
  ga.A = a; ga.B0 = b_hi; ga.B1 = b_lo;
  ga.M = int(m); ga.N = int(n); ga.K = int(k); ga.lda = lda; ga.ldb = ldb;
  ga.s_a = s_a; ga.s_0 = s_hi; ga.s_1 = s_lo;
  ga.out = grad; ga.ldo = n;
  ga.aux = dgelu;
  ga.part = static_cast<uint32_t*>(workspace);
  ga.cs_part = sums ? static_cast<float*>(colsum_ws) : nullptr;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool narrow = dgelu_narrow_eligible(ga);
  if (b_lo && a_fmt == TCFP_FP8_E5M2 && b_fmt == TCFP_FP8_E4M3 && m > 0 &&
      (narrow || persist_eligible(ga)) && num_cus() <= tcfp::max_parts()) {
    ga.tiles_m = int(m / 256);
    ga.tiles_n = int(n / (narrow ? 64 : 128));
    int r = launch_persist_gelu<2>(ga, narrow, st);
    if (r != TCFP_OK) return r;
    r = tcfp::quantize_with_parts(grad, TCFP_DTYPE_F32, m, n, fp8_fmt, q, q_t, inv_out, workspace,
                                  nullptr, nullptr, stream, num_cus(), false);
    if (r != TCFP_OK || !sums) return r;
    return tcfp::colsum_finalize(static_cast<const float*>(colsum_ws), m / kColGroup, n, col_sum,
                                 stream);
  }
  // any other shape: the GEMM into grad, then grad *= dgelu with the amax,
  // then the quantising pass with the column sums
  const int r = tcfp_dual_gemm(a, a_fmt, lda, b_hi, b_lo, b_fmt, ldb, m, n, k, s_a, s_hi, s_lo,
                               nullptr, grad, TCFP_DTYPE_F32, n, stream);
  if (r != TCFP_OK) return r;
  return tcfp::mul_quantize_colsum(grad, dgelu, m, n, fp8_fmt, grad, q, q_t, inv_out,
                                   sums ? col_sum : nullptr, workspace,
                                   static_cast<float*>(colsum_ws), stream);
}

extern "C" int tcfp_block_dual_gemm(const uint8_t* a, int a_fmt, int64_t lda, const int8_t* e_a,
                                    const uint8_t* b_hi, const uint8_t* b_lo, int b_fmt,
                                    int64_t ldb, const int8_t* e_hi, const int8_t* e_lo,
                                    int64_t m, int64_t n, int64_t k, int block,
                                    const float* bias, void* out, int out_dtype, int64_t ldo,
                                    void* stream) {
  const int rc = check_common(m, n, k, lda, ldb, ldo, a, b_hi, b_lo, out_dtype);
  if (rc != TCFP_OK) return rc;
  if (block != 32 && block != 64 && block != 128) return TCFP_ERR_SHAPE;
  if (k % block != 0) return TCFP_ERR_SHAPE;
  if (!e_a || !e_hi || (b_lo && !e_lo)) return TCFP_ERR_SHAPE;
  if (m == 0 || n == 0) return TCFP_OK;
  GemmArgs ga{};
  ga.A = a; ga.B0 = b_hi; ga.B1 = b_lo ? b_lo : b_hi;
  ga.M = int(m); ga.N = int(n); ga.K = int(k); ga.lda = lda; ga.ldb = ldb;
  ga.e_a = e_a; ga.e_0 = e_hi; ga.e_1 = b_lo ? e_lo : e_hi;
  ga.bs_shift = block == 32 ? 5 : (block == 64 ? 6 : 7);
  ga.bias = bias; ga.out = out; ga.ldo = ldo;
  return dispatch_all<1>(a_fmt, b_fmt, b_lo != nullptr, out_dtype, ga,
                         static_cast<hipStream_t>(stream));
}

namespace {

// The fused activation-quant GEMM: one launch of the 128 x 64 tile with the
// activation block-quantised inside (AQ 1 bf16 / 2 fp32, BSH = log2 block).
template <int AQ, int BSH>
int launch_actq(GemmArgs ga, hipStream_t st) {
  // fp32 activations always, bf16 ones when 128-row tiles would leave CUs
  // idle: 64-row tiles (twice the workgroups, half the quantisation per
  // workgroup and stage)
  const bool rows64 = AQ == 2 || int64_t((ga.M + 127) / 128) * ((ga.N + 63) / 64) < 2 * num_cus();
  const int BMv = rows64 ? 64 : 128;
  ga.tiles_m = (ga.M + BMv - 1) / BMv;
  ga.tiles_n = (ga.N + 63) / 64;
  if (!grid_x_fits(int64_t(ga.tiles_m) * ga.tiles_n, 256)) return TCFP_ERR_SHAPE;
  const dim3 grid(unsigned(ga.tiles_m) * unsigned(ga.tiles_n));
  if (rows64)
    gemm_nt_dma_kernel<0, 0, false, float, 4, 64, 64, 1, 2, BSH, AQ><<<grid, 256, 0, st>>>(ga);
  else if constexpr (AQ == 1)
    gemm_nt_dma_kernel<0, 0, false, float, 4, 128, 64, 1, 2, BSH, AQ><<<grid, 256, 0, st>>>(ga);
  return hipGetLastError() == hipSuccess ? TCFP_OK : TCFP_ERR_HIP;
}

}  // namespace

extern "C" int tcfp_act_quant_block_dual_gemm(const void* act, int act_dtype, int64_t lda,
                                              const uint8_t* w_hi, const uint8_t* w_lo,
                                              int64_t ldb, const int8_t* e_hi,
                                              const int8_t* e_lo, int64_t m, int64_t n,
                                              int64_t k, int block, const float* bias,
                                              float* out, int64_t ldo, uint8_t* act_fp8,
                                              int8_t* act_scales, void* stream) {
  if (act_dtype != TCFP_DTYPE_F32 && act_dtype != TCFP_DTYPE_BF16) return TCFP_ERR_DTYPE;
  if (m < 0 || n < 0 || k < 0 || m > INT32_MAX || n > INT32_MAX || k > INT32_MAX)
    return TCFP_ERR_SHAPE;
  if (block != 32 && block != 64 && block != 128) return TCFP_ERR_SHAPE;
  if (k % block != 0 || lda < k || ldb < k || ldo < n) return TCFP_ERR_SHAPE;
  if ((act_fp8 == nullptr) != (act_scales == nullptr)) return TCFP_ERR_SHAPE;
  if (!w_hi || !w_lo || !e_hi || !e_lo) return TCFP_ERR_SHAPE;
  const int es = act_dtype == TCFP_DTYPE_F32 ? 4 : 2;
  if ((lda * es) % 16 != 0 || ldb % 16 != 0) return TCFP_ERR_ALIGN;
  if (!al16(act) || !al16(w_hi) || !al16(w_lo) || (act_fp8 && !al16(act_fp8)))
    return TCFP_ERR_ALIGN;
  if (bias && !al16(bias)) return TCFP_ERR_ALIGN;
  if (m == 0 || n == 0) return TCFP_OK;
  // the activation rows and the weight rows of a tile must lie within one
  // buffer descriptor's 32-bit reach
  if (int64_t(128) * lda * es + k * es >= kMaxSpan || int64_t(64) * ldb + k >= kMaxSpan)
    return TCFP_ERR_SHAPE;
  GemmArgs ga{};
  ga.A = static_cast<const uint8_t*>(act);
  ga.B0 = w_hi; ga.B1 = w_lo;
  ga.M = int(m); ga.N = int(n); ga.K = int(k); ga.lda = lda * es; ga.ldb = ldb;
  ga.e_0 = e_hi; ga.e_1 = e_lo;
  ga.bs_shift = block == 32 ? 5 : (block == 64 ? 6 : 7);
  ga.bias = bias; ga.out = out; ga.ldo = ldo;
  ga.q_out = act_fp8; ga.e_out = act_scales;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (act_dtype == TCFP_DTYPE_BF16) {
    if (block == 32) return launch_actq<1, 5>(ga, st);
    if (block == 64) return launch_actq<1, 6>(ga, st);
    return launch_actq<1, 7>(ga, st);
  }
  if (block == 32) return launch_actq<2, 5>(ga, st);
  if (block == 64) return launch_actq<2, 6>(ga, st);
  return launch_actq<2, 7>(ga, st);
}

extern "C" int tcfp_block_dual_gemm_f32s(const uint8_t* a, int a_fmt, int64_t lda,
                                         const float* s_a, const uint8_t* b_hi,
                                         const uint8_t* b_lo, int b_fmt, int64_t ldb,
                                         const float* s_hi, const float* s_lo, int64_t m,
                                         int64_t n, int64_t k, int block, const float* bias,
                                         void* out, int out_dtype, int64_t ldo, void* stream) {
  const int rc = check_common(m, n, k, lda, ldb, ldo, a, b_hi, b_lo, out_dtype);
  if (rc != TCFP_OK) return rc;
  if (block != 32 && block != 64 && block != 128) return TCFP_ERR_SHAPE;
  if (k % block != 0 || m % 4 != 0 || n % 4 != 0) return TCFP_ERR_SHAPE;
  if (!s_a || !s_hi || (b_lo && !s_lo)) return TCFP_ERR_SHAPE;
  if (!al16(s_a) || !al16(s_hi) || (b_lo && !al16(s_lo))) return TCFP_ERR_ALIGN;
  if (m == 0 || n == 0) return TCFP_OK;
  GemmArgs ga{};
  ga.A = a; ga.B0 = b_hi; ga.B1 = b_lo ? b_lo : b_hi;
  ga.M = int(m); ga.N = int(n); ga.K = int(k); ga.lda = lda; ga.ldb = ldb;
  ga.s_a = s_a; ga.s_0 = s_hi; ga.s_1 = b_lo ? s_lo : s_hi;
  ga.bs_shift = block == 32 ? 5 : (block == 64 ? 6 : 7);
  ga.bias = bias; ga.out = out; ga.ldo = ldo;
  return dispatch_all<2>(a_fmt, b_fmt, b_lo != nullptr, out_dtype, ga,
                         static_cast<hipStream_t>(stream));
}

// Weight quantisation + block dual GEMM (the reference's single-kernel
// fused_wtquant_block_scaled_dual_gemm_forward).  Quantising W inside the
// GEMM would repeat the amax/convert work in every M-tile workgroup; one
// streaming dual-quant pass (with the error update) followed by the GEMM
// reads W once and moves only the FP8 codes through HBM again.
extern "C" int tcfp_wtquant_block_dual_gemm(const uint8_t* a, int a_fmt, int64_t lda,
                                            const int8_t* e_a, const void* w, int w_dtype,
                                            int64_t m, int64_t n, int64_t k, int block,
                                            float* ef, int stochastic_lo, uint64_t seed,
                                            uint64_t offset, uint8_t* w_hi, uint8_t* w_lo,
                                            int8_t* e_hi, int8_t* e_lo, const float* bias,
                                            void* out, int out_dtype, int64_t ldo,
                                            void* stream) {
  if (!a || !e_a || !w || !w_hi || !w_lo || !e_hi || !e_lo) return TCFP_ERR_SHAPE;
  const int rc = check_common(m, n, k, lda, k, ldo, a, w_hi, w_lo, out_dtype);
  if (rc != TCFP_OK) return rc;
  if (block != 32 && block != 64 && block != 128) return TCFP_ERR_SHAPE;
  if (k % block != 0) return TCFP_ERR_SHAPE;
  const int q = tcfp_block_dual_quantize(w, w_dtype, n, k, block, ef, 1, stochastic_lo, seed,
                                         offset, w_hi, w_lo, e_hi, e_lo, stream);
  if (q != TCFP_OK) return q;
  return tcfp_block_dual_gemm(a, a_fmt, lda, e_a, w_hi, w_lo, TCFP_FP8_E4M3, k, e_hi, e_lo, m, n,
                              k, block, bias, out, out_dtype, ldo, stream);
}

extern "C" int tcfp_gemm_set_tile_policy(int policy) {
  if (policy < 0 || policy > 5) return TCFP_ERR_SHAPE;
  g_tile_policy = policy;
  return TCFP_OK;
}

// ===========================================================================
// Block-scaled dgrad (reference fused_block_scaled_dual_gemm_backward_dx)
// ===========================================================================
//
// dX[m, k] = sum_n deq(G)[m, n] * (deq(W_hi)[n, k] + deq(W_lo)[n, k]) where the
// W exponents vary per (k-block, n): along the contraction index n they
// change every element, which no per-32-K MFMA scale can express.  Every
// dequantised operand value fp8 * 2^e is exactly representable in bf16, so
// the operands are dequantised once into bf16 (G as is, W transposed to
// [D_in, D_out] so the contraction is contiguous) and multiplied on the
// bf16 MFMA with fp32 accumulation: every product is exact, which is at
// least as accurate as the reference's dequantise-then-tf32 dot.
namespace {

// out[r, c] = bf16(q[r, c] * 2^e[c / bs, r]); 8 elements per thread
// (one block, since bs >= 32 and c % 8 == 0).
template <int FMT>
__global__ __launch_bounds__(256) void dequant_rows_bf16_kernel(
    const uint8_t* __restrict__ q, const int8_t* __restrict__ e, int64_t rows, int64_t cols,
    int bs_shift, int zero_sentinel, uint16_t* __restrict__ out) {
  const int64_t nvec = rows * cols / 8;
  const int64_t stride = int64_t(gridDim.x) * 256;
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < nvec; i += stride) {
    const int64_t r = (i * 8) / cols, c = (i * 8) - r * cols;
    const int ex = e[(c >> bs_shift) * rows + r];
    const float sc = (zero_sentinel && ex == -128) ? 0.0f : exp2i(ex);
    const uint2 w = *reinterpret_cast<const uint2*>(q + i * 8);
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t word = j < 2 ? w.x : w.y;
      const float a = fp8_to_f32<FMT>((word >> (16 * (j & 1))) & 0xFFu) * sc;
      const float b = fp8_to_f32<FMT>((word >> (16 * (j & 1) + 8)) & 0xFFu) * sc;
      o[j] = uint32_t(f32_to_bf16_rne(a)) | (uint32_t(f32_to_bf16_rne(b)) << 16);
    }
    *reinterpret_cast<uint4*>(out + i * 8) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// Byte B of w decoded (the decoders take the byte select directly).
template <int FMT, int B>
TCFP_DEV float fp8_byte_to_f32(uint32_t w) {
  if constexpr (FMT == TCFP_FP8_E5M2) return __builtin_amdgcn_cvt_f32_bf8(int(w), B);
  else return __builtin_amdgcn_cvt_f32_fp8(int(w), B);
}

// The 16 codes of a 16-byte row piece times sc, as bf16, into column j of
// the transposing tile: tile[lc + j][lr].
template <int FMT>
TCFP_DEV void deq16_to_tile(const uint4 w, float sc, uint16_t (*tile)[64 + 2], int lc, int lr) {
  const uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    tile[lc + 4 * i + 0][lr] = f32_to_bf16_rne(fp8_byte_to_f32<FMT, 0>(words[i]) * sc);
    tile[lc + 4 * i + 1][lr] = f32_to_bf16_rne(fp8_byte_to_f32<FMT, 1>(words[i]) * sc);
    tile[lc + 4 * i + 2][lr] = f32_to_bf16_rne(fp8_byte_to_f32<FMT, 2>(words[i]) * sc);
    tile[lc + 4 * i + 3][lr] = f32_to_bf16_rne(fp8_byte_to_f32<FMT, 3>(words[i]) * sc);
  }
}

// out[c, r] = bf16(q[r * ldq + c] * 2^e[c / bs, r]) through a 64 x 64 LDS
// tile (c < cols: a column range of a wider q when ldq > cols).  vec: q is
// 16-byte aligned and ldq % 16 == 0, so a full tile's thread reads its 16
// codes (one exponent block: bs >= 32) with one load.
template <int FMT>
__global__ __launch_bounds__(256) void dequant_t_bf16_kernel(
    const uint8_t* __restrict__ q0, const int8_t* __restrict__ e0, uint16_t* __restrict__ out0,
    const uint8_t* __restrict__ q1, const int8_t* __restrict__ e1, uint16_t* __restrict__ out1,
    int64_t rows, int64_t cols, int bs_shift, int64_t ldq, bool vec) {
  // blockIdx.y 0: matrix 0 (W_hi); 1: matrix 1 (W_lo, whose -128 exponent
  // marks a zero block)
  const bool second = blockIdx.y == 1;
  const uint8_t* __restrict__ q = second ? q1 : q0;
  const int8_t* __restrict__ e = second ? e1 : e0;
  uint16_t* __restrict__ out = second ? out1 : out0;
  const int zero_sentinel = second ? 1 : 0;
  __shared__ uint16_t tile[64][64 + 2];
  const int tiles_c = int((cols + 63) / 64);
  const int64_t r0 = int64_t(blockIdx.x / tiles_c) * 64, c0 = int64_t(blockIdx.x % tiles_c) * 64;
  const int t = threadIdx.x;
  if (vec && r0 + 64 <= rows && c0 + 64 <= cols) {
    const int lr = t >> 2, lc = (t & 3) * 16;
    const int64_t r = r0 + lr;
    const uint4 w = *reinterpret_cast<const uint4*>(q + r * ldq + c0 + lc);
    const int ex = e[((c0 + lc) >> bs_shift) * rows + r];
    deq16_to_tile<FMT>(w, (zero_sentinel && ex == -128) ? 0.0f : exp2i(ex), tile, lc, lr);
  } else {
    const int lr = t >> 2, lc = (t & 3) * 16;
    const int64_t r = r0 + lr;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int64_t c = c0 + lc + j;
      uint16_t v = 0;
      if (r < rows && c < cols) {
        const int ex = e[(c >> bs_shift) * rows + r];
        const float sc = (zero_sentinel && ex == -128) ? 0.0f : exp2i(ex);
        v = f32_to_bf16_rne(fp8_to_f32<FMT>(q[r * ldq + c]) * sc);
      }
      tile[lc + j][lr] = v;
    }
  }
  __syncthreads();
  {
    const int lc = t >> 2, lr = (t & 3) * 16;
    const int64_t c = c0 + lc;
    if (c < cols) {
      uint16_t* o = out + c * rows + r0 + lr;
      if ((rows % 8) == 0 && r0 + lr + 16 <= rows) {
        uint32_t w[8];
#pragma unroll
        for (int j = 0; j < 8; ++j)
          w[j] = uint32_t(tile[lc][lr + 2 * j]) | (uint32_t(tile[lc][lr + 2 * j + 1]) << 16);
        reinterpret_cast<uint4*>(o)[0] = make_uint4(w[0], w[1], w[2], w[3]);
        reinterpret_cast<uint4*>(o)[1] = make_uint4(w[4], w[5], w[6], w[7]);
      } else {
        for (int j = 0; j < 16; ++j)
          if (r0 + lr + j < rows) o[j] = tile[lc][lr + j];
      }
    }
  }
}

size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

// ---- block wgrad operands ------------------------------------------------
// dW[n, k] = sum_m g[m, n] * deq(x)[m, k] with fp32 g.  g is split into
// g_hi = bf16(g) and g_lo = bf16(g - g_hi) (together ~16 significant bits,
// relative error <= 2^-17), the dequantised activation is exact in bf16,
// and the two products are one bf16 GEMM over the concatenated contraction:
//   A' = [g_hi^T | g_lo^T]  [N, 2M],   B' = [x^T | x^T]  [K, 2M].

// A'[c, r] = hi(g[r, c]), A'[c, M + r] = lo(g[r, c]); g [rows, cols] fp32.
__global__ __launch_bounds__(256) void split_t_bf16_kernel(const float* __restrict__ g,
                                                           int64_t rows, int64_t cols,
                                                           uint16_t* __restrict__ out) {
  __shared__ float tile[64][64 + 1];
  const int tiles_c = int((cols + 63) / 64);
  const int64_t r0 = int64_t(blockIdx.x / tiles_c) * 64, c0 = int64_t(blockIdx.x % tiles_c) * 64;
  const int t = threadIdx.x;
  {
    const int lr = t >> 2, lc = (t & 3) * 16;
    const int64_t r = r0 + lr;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int64_t c = c0 + lc + j;
      tile[lc + j][lr] = (r < rows && c < cols) ? g[r * cols + c] : 0.0f;
    }
  }
  __syncthreads();
  const int lc = t >> 2, lr = (t & 3) * 16;
  const int64_t c = c0 + lc;
  if (c >= cols) return;
  uint16_t hi[16], lo[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const float v = tile[lc][lr + j];
    hi[j] = f32_to_bf16_rne(v);
    lo[j] = f32_to_bf16_rne(__fsub_rn(v, bf16_to_f32(hi[j])));
  }
  uint16_t* oh = out + c * (2 * rows) + r0 + lr;
  uint16_t* ol = oh + rows;
  if ((rows % 8) == 0 && r0 + lr + 16 <= rows) {
    uint32_t wh[8], wl[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      wh[j] = uint32_t(hi[2 * j]) | (uint32_t(hi[2 * j + 1]) << 16);
      wl[j] = uint32_t(lo[2 * j]) | (uint32_t(lo[2 * j + 1]) << 16);
    }
    reinterpret_cast<uint4*>(oh)[0] = make_uint4(wh[0], wh[1], wh[2], wh[3]);
    reinterpret_cast<uint4*>(oh)[1] = make_uint4(wh[4], wh[5], wh[6], wh[7]);
    reinterpret_cast<uint4*>(ol)[0] = make_uint4(wl[0], wl[1], wl[2], wl[3]);
    reinterpret_cast<uint4*>(ol)[1] = make_uint4(wl[4], wl[5], wl[6], wl[7]);
  } else {
    for (int j = 0; j < 16; ++j)
      if (r0 + lr + j < rows) { oh[j] = hi[j]; ol[j] = lo[j]; }
  }
}

// B'[c, r] = bf16(q[r * ldq + c] * 2^e[c / bs, r]) (exact), and with dup
// also B'[c, M + r] (rows of 2M); c < cols.  vec as in dequant_t_bf16_kernel.
template <int FMT>
__global__ __launch_bounds__(256) void dequant_t_dup_bf16_kernel(
    const uint8_t* __restrict__ q, const int8_t* __restrict__ e, int64_t rows, int64_t cols,
    int bs_shift, uint16_t* __restrict__ out, int64_t ldq, bool dup, bool vec) {
  __shared__ uint16_t tile[64][64 + 2];
  const int tiles_c = int((cols + 63) / 64);
  const int64_t r0 = int64_t(blockIdx.x / tiles_c) * 64, c0 = int64_t(blockIdx.x % tiles_c) * 64;
  const int t = threadIdx.x;
  if (vec && r0 + 64 <= rows && c0 + 64 <= cols) {
    const int lr = t >> 2, lc = (t & 3) * 16;
    const int64_t r = r0 + lr;
    const uint4 w = *reinterpret_cast<const uint4*>(q + r * ldq + c0 + lc);
    deq16_to_tile<FMT>(w, exp2i(e[((c0 + lc) >> bs_shift) * rows + r]), tile, lc, lr);
  } else {
    const int lr = t >> 2, lc = (t & 3) * 16;
    const int64_t r = r0 + lr;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int64_t c = c0 + lc + j;
      uint16_t v = 0;
      if (r < rows && c < cols)
        v = f32_to_bf16_rne(fp8_to_f32<FMT>(q[r * ldq + c]) * exp2i(e[(c >> bs_shift) * rows + r]));
      tile[lc + j][lr] = v;
    }
  }
  __syncthreads();
  const int lc = t >> 2, lr = (t & 3) * 16;
  const int64_t c = c0 + lc;
  if (c >= cols) return;
  uint16_t* o0 = out + c * (dup ? 2 * rows : rows) + r0 + lr;
  uint16_t* o1 = o0 + rows;
  if ((rows % 8) == 0 && r0 + lr + 16 <= rows) {
    uint32_t w[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      w[j] = uint32_t(tile[lc][lr + 2 * j]) | (uint32_t(tile[lc][lr + 2 * j + 1]) << 16);
    reinterpret_cast<uint4*>(o0)[0] = make_uint4(w[0], w[1], w[2], w[3]);
    reinterpret_cast<uint4*>(o0)[1] = make_uint4(w[4], w[5], w[6], w[7]);
    if (dup) {
      reinterpret_cast<uint4*>(o1)[0] = make_uint4(w[0], w[1], w[2], w[3]);
      reinterpret_cast<uint4*>(o1)[1] = make_uint4(w[4], w[5], w[6], w[7]);
    }
  } else {
    for (int j = 0; j < 16; ++j)
      if (r0 + lr + j < rows) {
        o0[j] = tile[lc][lr + j];
        if (dup) o1[j] = tile[lc][lr + j];
      }
  }
}

}  // namespace

namespace {

// Dequantised bf16 operand copies of the block backward are made in column
// chunks whose copies stay within this many bytes (the GEMMs run per chunk
// into a column range of the output), so the workspace does not grow with
// the layer; a chunk keeps at least 256 columns.
constexpr int64_t kOperandChunkBytes = int64_t(64) << 20;

int64_t chunk_cols(int64_t bytes_per_col, int64_t cols) {
  int64_t c = kOperandChunkBytes / std::max<int64_t>(bytes_per_col, 1) / 256 * 256;
  c = std::max<int64_t>(c, 256);
  return std::min(c, cols);
}

// dx columns per dgrad chunk: W_hi^T and W_lo^T rows of d_out bf16 each
int64_t dgrad_chunk(int64_t d_out, int64_t d_in) { return chunk_cols(4 * d_out, d_in); }

// Per chunk of dx columns [c0, c0 + n): W_hi^T, W_lo^T rows c0.. dequantised
// into bf16 (one launch), then the bf16 dual GEMM A = G [m, d_out] x
// B = W^T [n, d_out] (K counts bytes) into dx[:, c0 ..] (fp32, ld d_in).
int dgrad_bf16(const uint16_t* gd, const uint8_t* w_hi, const uint8_t* w_lo, const int8_t* e_hi,
               const int8_t* e_lo, int64_t m, int64_t d_out, int64_t d_in, int shift, float* dx,
               uint16_t* wth, uint16_t* wtl, hipStream_t st) {
  const int64_t cw = dgrad_chunk(d_out, d_in);
  for (int64_t c0 = 0; c0 < d_in; c0 += cw) {
    const int64_t n = std::min(cw, d_in - c0);
    const int64_t tiles = ((d_out + 63) / 64) * ((n + 63) / 64);
    if (!grid_x_fits(tiles, 256)) return TCFP_ERR_SHAPE;
    const int64_t eo = (c0 >> shift) * d_out;  // c0 is a multiple of the block
    const bool vec = al16(w_hi + c0) && (!w_lo || al16(w_lo + c0)) && d_in % 16 == 0;
    dequant_t_bf16_kernel<TCFP_FP8_E4M3><<<dim3(unsigned(tiles), w_lo ? 2u : 1u), 256, 0, st>>>(
        w_hi + c0, e_hi + eo, wth, w_lo ? w_lo + c0 : nullptr, w_lo ? e_lo + eo : nullptr, wtl,
        d_out, n, shift, d_in, vec);
    if (hipGetLastError() != hipSuccess) return TCFP_ERR_HIP;
    GemmArgs ga{};
    ga.A = reinterpret_cast<const uint8_t*>(gd);
    ga.B0 = reinterpret_cast<const uint8_t*>(wth);
    ga.B1 = reinterpret_cast<const uint8_t*>(w_lo ? wtl : wth);
    ga.M = int(m); ga.N = int(n); ga.K = int(2 * d_out);
    ga.lda = 2 * d_out; ga.ldb = 2 * d_out;
    ga.out = dx + c0; ga.ldo = d_in;
    const int rc = w_lo ? launch_gemm<kBF16, kBF16, false, float, 0>(ga, st)
                        : launch_gemm<kBF16, kBF16, true, float, 0>(ga, st);
    if (rc != TCFP_OK) return rc;
  }
  return TCFP_OK;
}

size_t dgrad_copy_bytes(int64_t d_out, int64_t d_in) {
  return align256(size_t(dgrad_chunk(d_out, d_in)) * size_t(d_out) * 2);
}

}  // namespace

extern "C" size_t tcfp_block_dual_gemm_dx_workspace_bytes(int64_t m, int64_t d_out, int64_t d_in) {
  if (m < 0 || d_out < 0 || d_in < 0) return 0;
  return align256(size_t(m) * size_t(d_out) * 2) + 2 * dgrad_copy_bytes(d_out, d_in);
}

extern "C" int tcfp_block_dual_gemm_dx(const uint8_t* g, int g_fmt, const int8_t* e_g,
                                       const uint8_t* w_hi, const uint8_t* w_lo,
                                       const int8_t* e_hi, const int8_t* e_lo, int64_t m,
                                       int64_t d_out, int64_t d_in, int block, float* dx,
                                       void* workspace, size_t workspace_bytes, void* stream) {
  if (m < 0 || d_out < 0 || d_in < 0 || m > INT32_MAX || d_in > INT32_MAX ||
      2 * d_out > INT32_MAX)
    return TCFP_ERR_SHAPE;
  if (block != 32 && block != 64 && block != 128) return TCFP_ERR_SHAPE;
  if (d_out % block != 0 || d_in % block != 0) return TCFP_ERR_SHAPE;
  if (g_fmt != TCFP_FP8_E4M3 && g_fmt != TCFP_FP8_E5M2) return TCFP_ERR_DTYPE;
  if (!g || !e_g || !w_hi || !e_hi || (w_lo && !e_lo) || !dx) return TCFP_ERR_SHAPE;
  if (m == 0 || d_in == 0) return TCFP_OK;
  if (!workspace || workspace_bytes < tcfp_block_dual_gemm_dx_workspace_bytes(m, d_out, d_in))
    return TCFP_ERR_WORKSPACE;
  if (!al16(workspace) || !al16(dx)) return TCFP_ERR_ALIGN;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int shift = block == 32 ? 5 : (block == 64 ? 6 : 7);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  uint16_t* gd = reinterpret_cast<uint16_t*>(ws);
  uint16_t* wth = reinterpret_cast<uint16_t*>(ws + align256(size_t(m) * size_t(d_out) * 2));
  uint16_t* wtl = reinterpret_cast<uint16_t*>(reinterpret_cast<uint8_t*>(wth) +
                                              dgrad_copy_bytes(d_out, d_in));
  // dequantised operands
  {
    const int64_t nvec = m * d_out / 8;
    int64_t gr = (nvec + 255) / 256;
    gr = gr > int64_t(num_cus()) * 8 ? int64_t(num_cus()) * 8 : (gr < 1 ? 1 : gr);
    if (g_fmt == TCFP_FP8_E5M2)
      dequant_rows_bf16_kernel<TCFP_FP8_E5M2><<<unsigned(gr), 256, 0, st>>>(g, e_g, m, d_out, shift, 0, gd);
    else
      dequant_rows_bf16_kernel<TCFP_FP8_E4M3><<<unsigned(gr), 256, 0, st>>>(g, e_g, m, d_out, shift, 0, gd);
    if (hipGetLastError() != hipSuccess) return TCFP_ERR_HIP;
  }
  return dgrad_bf16(gd, w_hi, w_lo, e_hi, e_lo, m, d_out, d_in, shift, dx, wth, wtl, st);
}

extern "C" size_t tcfp_block_dual_gemm_dx_bf16_workspace_bytes(int64_t d_out, int64_t d_in) {
  if (d_out < 0 || d_in < 0) return 0;
  return 2 * dgrad_copy_bytes(d_out, d_in);
}

extern "C" int tcfp_block_dual_gemm_dx_bf16(const uint16_t* g_deq, const uint8_t* w_hi,
                                            const uint8_t* w_lo, const int8_t* e_hi,
                                            const int8_t* e_lo, int64_t m, int64_t d_out,
                                            int64_t d_in, int block, float* dx, void* workspace,
                                            size_t workspace_bytes, void* stream) {
  if (m < 0 || d_out < 0 || d_in < 0 || m > INT32_MAX || d_in > INT32_MAX ||
      2 * d_out > INT32_MAX)
    return TCFP_ERR_SHAPE;
  if (block != 32 && block != 64 && block != 128) return TCFP_ERR_SHAPE;
  if (d_out % block != 0 || d_in % block != 0) return TCFP_ERR_SHAPE;
  if (!g_deq || !w_hi || !e_hi || (w_lo && !e_lo) || !dx) return TCFP_ERR_SHAPE;
  if (m == 0 || d_in == 0) return TCFP_OK;
  if (!workspace || workspace_bytes < tcfp_block_dual_gemm_dx_bf16_workspace_bytes(d_out, d_in))
    return TCFP_ERR_WORKSPACE;
  if (!al16(workspace) || !al16(dx) || !al16(g_deq)) return TCFP_ERR_ALIGN;
  const int shift = block == 32 ? 5 : (block == 64 ? 6 : 7);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  uint16_t* wth = reinterpret_cast<uint16_t*>(ws);
  uint16_t* wtl = reinterpret_cast<uint16_t*>(ws + dgrad_copy_bytes(d_out, d_in));
  return dgrad_bf16(g_deq, w_hi, w_lo, e_hi, e_lo, m, d_out, d_in, shift, dx, wth, wtl,
                    static_cast<hipStream_t>(stream));
}

namespace {

// dw[i] = sum_s part[s * stride + i], summed in split order (deterministic);
// four fp32 per thread (n4 = elements / 4; stride % 4 == 0).
// The partials are [rows, cols] row-major per split (cols % 4 == 0); out
// has row stride ldo.
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ part,
                                                            int splits, int64_t n4,
                                                            int64_t stride, int64_t cols,
                                                            int64_t ldo,
                                                            float* __restrict__ out) {
  const int64_t step = int64_t(gridDim.x) * 256;
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < n4; i += step) {
    float4 a = reinterpret_cast<const float4*>(part)[i];
    for (int sp = 1; sp < splits; ++sp) {
      const float4 b = reinterpret_cast<const float4*>(part + sp * stride)[i];
      a.x += b.x; a.y += b.y; a.z += b.z; a.w += b.w;
    }
    const int64_t e = 4 * i, r = e / cols, c = e - r * cols;
    *reinterpret_cast<float4*>(out + r * ldo + c) = a;
  }
}

// Split-K factor of the block wgrad GEMM (contraction 2m bf16 = 4m bytes;
// m bf16 = 2m bytes without the low half, `lo` false): when the [n_out,
// k_in] output gives at most half the CUs a 128 x 128 tile, split the
// contraction so every CU gets a workgroup, keeping at least four 128-byte
// stages per split.  Returns the split count and sets *kc to the split
// length in bytes (a multiple of 128).
int64_t wgrad_splits(int64_t m, int64_t n_out, int64_t k_in, int64_t* kc, bool lo = true) {
  const int64_t kbytes = (lo ? 4 : 2) * m;
  *kc = kbytes;
  const int64_t tiles = ((n_out + 127) / 128) * ((k_in + 127) / 128);
  const int64_t cus = num_cus();
  if (tiles <= 0 || 2 * tiles > cus) return 1;
  const int64_t s = std::min((cus + tiles - 1) / tiles, kbytes / 512);
  if (s < 2) return 1;
  *kc = ((kbytes + s - 1) / s + 127) / 128 * 128;
  return (kbytes + *kc - 1) / *kc;
}

// The wgrad GEMM over the concatenated contraction: A' = [g_hi | g_lo]^T
// [n_out, 2m], B' = [x | x]^T [k_in, 2m] (bf16; with `wrap` one copy
// x^T [k_in, m] read twice), dw [n_out, k_in] fp32 with row stride ldo;
// split-K partials go to `part` when the output is small.  Without the low
// half (`lo` false): A' = g_hi^T [n_out, m] against one copy x^T [k_in, m].
int wgrad_gemm(const uint16_t* ap, const uint16_t* bp, int64_t m, int64_t n_out, int64_t k_in,
               float* dw, int64_t ldo, float* part, bool wrap, hipStream_t st, bool lo = true) {
  GemmArgs ga{};
  ga.A = reinterpret_cast<const uint8_t*>(ap);
  ga.B0 = reinterpret_cast<const uint8_t*>(bp);
  ga.B1 = ga.B0;
  ga.M = int(n_out); ga.N = int(k_in);
  if (lo) {
    ga.K = int(4 * m);  // bytes of 2M bf16
    ga.lda = 4 * m; ga.ldb = wrap ? 2 * m : 4 * m;
    ga.kwrap_b = wrap ? int(2 * m) : 0;
  } else {
    ga.K = int(2 * m);
    ga.lda = 2 * m; ga.ldb = 2 * m;
    ga.kwrap_b = 0;
  }
  ga.out = dw; ga.ldo = ldo;
  int64_t kc;
  const int64_t splits = wgrad_splits(m, n_out, k_in, &kc, lo);
  if (splits <= 1) return launch_gemm<kBF16, kBF16, true, float, 0>(ga, st);
  // partial products of each K chunk ([n_out, k_in] each), then their sum
  // in split order
  ga.out = part;
  ga.ldo = k_in;
  ga.kc = int(kc);
  ga.split_stride = n_out * k_in;
  const int rc = launch_gemm<kBF16, kBF16, true, float, 0>(ga, st);
  if (rc != TCFP_OK) return rc;
  const int64_t n4 = n_out * k_in / 4;
  const int blocks = int(std::min<int64_t>((n4 + 255) / 256, int64_t(num_cus()) * 8));
  splitk_reduce_kernel<<<blocks, 256, 0, st>>>(part, int(splits), n4, n_out * k_in, k_in, ldo,
                                               dw);
  return hipGetLastError() == hipSuccess ? TCFP_OK : TCFP_ERR_HIP;
}

// One copy of x^T serves both halves of the contraction when its rows (m
// bf16 = 2m bytes) are whole 128-byte stages.
bool wgrad_wrap(int64_t m) { return m > 0 && (2 * m) % kSK == 0; }
// x^T copy rows: m bf16 (one copy serves both halves, or there is no low
// half), 2m otherwise
bool wgrad_one_copy(int64_t m, bool lo) { return !lo || wgrad_wrap(m); }
// dw columns per wgrad chunk
int64_t wgrad_chunk(int64_t m, int64_t k_in, bool lo = true) {
  return chunk_cols((wgrad_one_copy(m, lo) ? 2 : 4) * std::max<int64_t>(m, 1), k_in);
}
size_t wgrad_part_bytes(int64_t m, int64_t n_out, int64_t cols, bool lo = true) {
  int64_t kc;
  const int64_t splits = wgrad_splits(m, n_out, cols, &kc, lo);
  return splits > 1 ? align256(size_t(splits) * size_t(n_out) * size_t(cols) * 4) : 0;
}
// Workspace of the chunked wgrad: one chunk's x^T copy, then the partials.
size_t wgrad_copy_bytes(int64_t m, int64_t k_in, bool lo = true) {
  return align256(size_t(wgrad_chunk(m, k_in, lo)) * size_t(wgrad_one_copy(m, lo) ? m : 2 * m) *
                  2);
}
size_t wgrad_ws_bytes(int64_t m, int64_t n_out, int64_t k_in, bool lo = true) {
  const int64_t kw = wgrad_chunk(m, k_in, lo);
  const int64_t rem = kw > 0 ? k_in % kw : 0;
  return wgrad_copy_bytes(m, k_in, lo) +
         std::max(wgrad_part_bytes(m, n_out, kw, lo),
                  rem ? wgrad_part_bytes(m, n_out, rem, lo) : 0);
}

// dw = A'^T-product of the split gradient ap ([n_out, 2m] bf16; [n_out, m]
// without the low half) with the dequantised activation, per chunk of dw
// columns: x^T rows c0.. dequantised into the workspace, then the GEMM into
// dw[:, c0 ..].
int wgrad_chunked(const uint16_t* ap, int64_t m, int64_t n_out, const uint8_t* x, int x_fmt,
                  const int8_t* e_x, int64_t k_in, int shift, float* dw, uint8_t* ws,
                  hipStream_t st, bool lo = true) {
  const bool wrap = wgrad_wrap(m);
  const bool dup = !wgrad_one_copy(m, lo);
  const int64_t kw = wgrad_chunk(m, k_in, lo);
  uint16_t* bp = reinterpret_cast<uint16_t*>(ws);
  float* part = reinterpret_cast<float*>(ws + wgrad_copy_bytes(m, k_in, lo));
  for (int64_t c0 = 0; c0 < k_in; c0 += kw) {
    const int64_t n = std::min(kw, k_in - c0);
    if (m > 0) {
      const int64_t tx = ((m + 63) / 64) * ((n + 63) / 64);
      if (!grid_x_fits(tx, 256)) return TCFP_ERR_SHAPE;
      const int64_t eo = (c0 >> shift) * m;  // c0 is a multiple of the block
      const bool vec = al16(x + c0) && k_in % 16 == 0;
      if (x_fmt == TCFP_FP8_E5M2)
        dequant_t_dup_bf16_kernel<TCFP_FP8_E5M2><<<unsigned(tx), 256, 0, st>>>(
            x + c0, e_x + eo, m, n, shift, bp, k_in, dup, vec);
      else
        dequant_t_dup_bf16_kernel<TCFP_FP8_E4M3><<<unsigned(tx), 256, 0, st>>>(
            x + c0, e_x + eo, m, n, shift, bp, k_in, dup, vec);
      if (hipGetLastError() != hipSuccess) return TCFP_ERR_HIP;
    }
    const int rc = wgrad_gemm(ap, bp, m, n_out, n, dw + c0, k_in, part, wrap, st, lo);
    if (rc != TCFP_OK) return rc;
  }
  return TCFP_OK;
}

// ---- fused gradient preparation for the block backward ---------------------
// One pass over the fp32 gradient g [m, n] in 64 x 128 tiles writes, as
// requested:
//  * gd [m, n] bf16: g block-quantised to E5M2 per (row, n-block) with the
//    exponent rule of block_quantize_fp8 (tcfp/kernels.py:205-275) and
//    dequantised -- the dgrad's G operand;
//  * gs [n, 2m] bf16: [bf16(g) | bf16(g - bf16(g))] transposed -- the
//    wgrad's split gradient (with `lo` false gs [n, m]: bf16(g) transposed,
//    the single-pass wgrad's operand);
//  * cpart [ceil(m/64), n] fp32: per-tile column sums (the bias gradient
//    after colsum_tiles_kernel).
// n % 32 == 0 (the block sizes divide it).
template <int BS>
__global__ __launch_bounds__(256) void grad_prep_kernel(const float* __restrict__ g, int64_t m,
                                                        int64_t n, uint16_t* __restrict__ gd,
                                                        uint16_t* __restrict__ gs,
                                                        float* __restrict__ cpart,
                                                        uint8_t* __restrict__ gq,
                                                        int8_t* __restrict__ ge, bool grouped,
                                                        bool lo) {
  __shared__ float tile[128][64 + 1];  // [column][row]
  const int tiles_c = int((n + 127) / 128);
  int64_t tr, c0;
  if (grouped) {
    // XCD-contiguous runs (workgroup b on XCD b % 8 takes item
    // (b % 8) * T/8 + b / 8) over groups of 16 row tiles, column tiles
    // fastest within a group: the workgroups resident at once cover
    // 16 x 64 rows of g and a 16 x 64-row band of each gs row they write,
    // instead of one band of every gs row (8192 x 16384: 333 -> 246 us)
    const int tiles_r = int((m + 63) / 64);
    const uint32_t T = gridDim.x, bb = blockIdx.x;
    const uint32_t b = (T & 7u) == 0 ? (bb & 7u) * (T >> 3) + (bb >> 3) : bb;
    constexpr int GR = 16;
    const int per = GR * tiles_c;
    const int fr = int(b / per) * GR;
    const int gr = min(tiles_r - fr, GR);
    tr = fr + int(b % per) % gr;
    c0 = int64_t(int(b % per) / gr) * 128;
  } else {
    tr = blockIdx.x / tiles_c;
    c0 = int64_t(blockIdx.x % tiles_c) * 128;
  }
  const int64_t r0 = tr * 64;
  const int t = threadIdx.x;
  // phase 1: row r0 + t/4, columns c0 + 32*(t%4) .. +31 (one 32-wide segment)
  const int lr = t >> 2, seg = t & 3;
  const int64_t r = r0 + lr, cb = c0 + seg * 32;
  const bool in = r < m && cb < n;
  float v[32];
  if (in) {
#pragma unroll
    for (int j = 0; j < 32; j += 4) {
      const float4 a = *reinterpret_cast<const float4*>(g + r * n + cb + j);
      v[j] = a.x; v[j + 1] = a.y; v[j + 2] = a.z; v[j + 3] = a.w;
    }
  } else {
#pragma unroll
    for (int j = 0; j < 32; ++j) v[j] = 0.0f;
  }
  if (gd || gq) {
    // block amax: a 32-wide segment per lane; 64 / 128-wide blocks span
    // the 2 / 4 lanes of the same row
    uint32_t a = 0;
#pragma unroll
    for (int j = 0; j < 32; ++j) a = a > (__float_as_uint(v[j]) & 0x7FFFFFFFu) ? a : (__float_as_uint(v[j]) & 0x7FFFFFFFu);
    if constexpr (BS >= 64) { const uint32_t o = __shfl_xor(a, 1, 64); a = a > o ? a : o; }
    if constexpr (BS >= 128) { const uint32_t o = __shfl_xor(a, 2, 64); a = a > o ? a : o; }
    const int e = block_exponent(__uint_as_float(a), kE5M2Max);
    const float mul = exp2i(-e), sc = exp2i(e);
    uint32_t w[16], cw[8];
#pragma unroll
    for (int j = 0; j < 32; j += 4) {
      float c4[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float x = v[j + q] * mul;
        c4[q] = x > kE5M2Max ? kE5M2Max : (x < -kE5M2Max ? -kE5M2Max : x);
      }
      const uint32_t codes = cvt4_fp8<TCFP_FP8_E5M2>(c4[0], c4[1], c4[2], c4[3]);
      cw[j / 4] = codes;
      uint16_t b[4];
#pragma unroll
      for (int q = 0; q < 4; ++q)
        b[q] = f32_to_bf16_rne(fp8_to_f32<TCFP_FP8_E5M2>((codes >> (8 * q)) & 0xFFu) * sc);
      w[j / 2] = uint32_t(b[0]) | (uint32_t(b[1]) << 16);
      w[j / 2 + 1] = uint32_t(b[2]) | (uint32_t(b[3]) << 16);
    }
    if (in && gd) {
      uint4* o = reinterpret_cast<uint4*>(gd + r * n + cb);
#pragma unroll
      for (int q = 0; q < 4; ++q) o[q] = make_uint4(w[4 * q], w[4 * q + 1], w[4 * q + 2], w[4 * q + 3]);
    }
    if (in && gq) {
      // the E5M2 codes [m, n] and the block exponents [n / BS, m] (the lane
      // at the block's first segment writes it)
      uint4* o = reinterpret_cast<uint4*>(gq + r * n + cb);
      o[0] = make_uint4(cw[0], cw[1], cw[2], cw[3]);
      o[1] = make_uint4(cw[4], cw[5], cw[6], cw[7]);
      if ((cb & (BS - 1)) == 0) ge[(cb / BS) * m + r] = int8_t(e);
    }
  }
  if (!gs && !cpart) return;
#pragma unroll
  for (int j = 0; j < 32; ++j) tile[seg * 32 + j][lr] = v[j];
  __syncthreads();
  // phase 2: column c0 + t/2, rows r0 + 32*(t%2) .. +31
  const int cc = t >> 1, half = t & 1;
  const int64_t c = c0 + cc;
  float sum = 0.0f;
  uint16_t hi[32], lo_v[32];
#pragma unroll
  for (int j = 0; j < 32; ++j) {
    const float x = tile[cc][half * 32 + j];
    sum += x;
    hi[j] = f32_to_bf16_rne(x);
    lo_v[j] = f32_to_bf16_rne(__fsub_rn(x, bf16_to_f32(hi[j])));
  }
  if (cpart) {
    const float other = __shfl_xor(sum, 1, 64);
    if (half == 0 && c < n) cpart[tr * n + c] = sum + other;
  }
  if (gs && c < n) {
    const int64_t rb = r0 + half * 32;
    uint16_t* oh = gs + c * (lo ? 2 * m : m) + rb;
    uint16_t* ol = oh + m;
    if ((m % 8) == 0 && rb + 32 <= m) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint32_t wh[4], wl[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          wh[j] = uint32_t(hi[8 * q + 2 * j]) | (uint32_t(hi[8 * q + 2 * j + 1]) << 16);
          wl[j] = uint32_t(lo_v[8 * q + 2 * j]) | (uint32_t(lo_v[8 * q + 2 * j + 1]) << 16);
        }
        reinterpret_cast<uint4*>(oh)[q] = make_uint4(wh[0], wh[1], wh[2], wh[3]);
        if (lo) reinterpret_cast<uint4*>(ol)[q] = make_uint4(wl[0], wl[1], wl[2], wl[3]);
      }
    } else {
      for (int j = 0; j < 32; ++j)
        if (rb + j < m) {
          oh[j] = hi[j];
          if (lo) ol[j] = lo_v[j];
        }
    }
  }
}

// out[c] = sum over row tiles of part[tile, c]: a workgroup takes 16
// columns, its 16 lanes per column sum the tiles t = lane, lane + 16, ... in
// order, and the 16 lane sums are added in lane order (a fixed order: the
// result is deterministic).  Sixteen-way parallel along the tiles, so the
// chain of dependent loads per thread is tiles / 16 long.
__global__ __launch_bounds__(256) void colsum_tiles_kernel(const float* __restrict__ part,
                                                           int64_t tiles, int64_t n,
                                                           float* __restrict__ out) {
  __shared__ float red[16][17];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int64_t c = int64_t(blockIdx.x) * 16 + tx;
  float s = 0.0f;
  if (c < n)
    for (int64_t t = ty; t < tiles; t += 16) s += part[t * n + c];
  red[ty][tx] = s;
  __syncthreads();
  if (ty == 0 && c < n) {
    float a = red[0][tx];
#pragma unroll
    for (int k = 1; k < 16; ++k) a += red[k][tx];
    out[c] = a;
  }
}

}  // namespace

extern "C" size_t tcfp_block_grad_prep_workspace_bytes(int64_t m, int64_t n) {
  if (m < 0 || n < 0) return 0;
  return align256(size_t((m + 63) / 64) * size_t(n) * 4);
}

extern "C" int tcfp_block_grad_prep(const float* g, int64_t m, int64_t n, int block,
                                    uint16_t* g_deq, uint16_t* g_split_t, int split_lo,
                                    float* bias_grad,
                                    uint8_t* g_fp8, int8_t* g_exps, void* workspace,
                                    size_t workspace_bytes, void* stream) {
  if (m < 0 || n < 0 || m > INT32_MAX || n > INT32_MAX) return TCFP_ERR_SHAPE;
  if (block != 32 && block != 64 && block != 128) return TCFP_ERR_SHAPE;
  if (n % block != 0) return TCFP_ERR_SHAPE;
  if (!g) return TCFP_ERR_SHAPE;
  if (bias_grad && (!workspace || workspace_bytes < tcfp_block_grad_prep_workspace_bytes(m, n)))
    return TCFP_ERR_WORKSPACE;
  if ((g_fp8 == nullptr) != (g_exps == nullptr)) return TCFP_ERR_SHAPE;
  if (split_lo != 0 && split_lo != 1) return TCFP_ERR_SHAPE;
  if (!al16(g) || (g_deq && !al16(g_deq)) || (g_split_t && !al16(g_split_t)) ||
      (g_fp8 && !al16(g_fp8)) || (workspace && !al16(workspace)))
    return TCFP_ERR_ALIGN;
  if (n == 0) return TCFP_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (m == 0) {
    if (bias_grad) {
      colsum_tiles_kernel<<<unsigned((n + 15) / 16), 256, 0, st>>>(nullptr, 0, n, bias_grad);
      return hipGetLastError() == hipSuccess ? TCFP_OK : TCFP_ERR_HIP;
    }
    return TCFP_OK;
  }
  const int64_t tr = (m + 63) / 64, tc = (n + 127) / 128;
  if (!grid_x_fits(tr * tc, 256)) return TCFP_ERR_SHAPE;
  float* part = bias_grad ? static_cast<float*>(workspace) : nullptr;
  const unsigned grid = unsigned(tr * tc);
  // wide gradients take the grouped tile order (measured: 26% faster at
  // n = 16384, the same at 4096, 8% slower at 1024)
  const bool grouped = n >= 8192;
  if (block == 32)
    grad_prep_kernel<32><<<grid, 256, 0, st>>>(g, m, n, g_deq, g_split_t, part, g_fp8, g_exps,
                                                  grouped, split_lo != 0);
  else if (block == 64)
    grad_prep_kernel<64><<<grid, 256, 0, st>>>(g, m, n, g_deq, g_split_t, part, g_fp8, g_exps,
                                                  grouped, split_lo != 0);
  else
    grad_prep_kernel<128><<<grid, 256, 0, st>>>(g, m, n, g_deq, g_split_t, part, g_fp8, g_exps,
                                                  grouped, split_lo != 0);
  if (bias_grad)
    colsum_tiles_kernel<<<unsigned((n + 15) / 16), 256, 0, st>>>(part, tr, n, bias_grad);
  return hipGetLastError() == hipSuccess ? TCFP_OK : TCFP_ERR_HIP;
}

extern "C" size_t tcfp_block_wgrad_workspace_bytes(int64_t m, int64_t n_out, int64_t k_in) {
  if (m < 0 || n_out < 0 || k_in < 0) return 0;
  return align256(size_t(n_out) * size_t(2 * m) * 2) + wgrad_ws_bytes(m, n_out, k_in);
}

extern "C" int tcfp_block_wgrad(const float* g, int64_t m, int64_t n_out, const uint8_t* x,
                                int x_fmt, const int8_t* e_x, int64_t k_in, int block, float* dw,
                                void* workspace, size_t workspace_bytes, void* stream) {
  if (m < 0 || n_out < 0 || k_in < 0 || n_out > INT32_MAX || k_in > INT32_MAX ||
      4 * m > INT32_MAX)
    return TCFP_ERR_SHAPE;
  if (block != 32 && block != 64 && block != 128) return TCFP_ERR_SHAPE;
  if (k_in % block != 0 || m % 4 != 0) return TCFP_ERR_SHAPE;
  if (x_fmt != TCFP_FP8_E4M3 && x_fmt != TCFP_FP8_E5M2) return TCFP_ERR_DTYPE;
  if (!g || !x || !e_x || !dw) return TCFP_ERR_SHAPE;
  if (n_out == 0 || k_in == 0) return TCFP_OK;
  if (!workspace || workspace_bytes < tcfp_block_wgrad_workspace_bytes(m, n_out, k_in))
    return TCFP_ERR_WORKSPACE;
  if (!al16(workspace) || !al16(dw)) return TCFP_ERR_ALIGN;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int shift = block == 32 ? 5 : (block == 64 ? 6 : 7);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  uint16_t* ap = reinterpret_cast<uint16_t*>(ws);
  if (m > 0) {  // (an empty contraction gives dW = 0 through the GEMM with K = 0)
    const int64_t tg = ((m + 63) / 64) * ((n_out + 63) / 64);
    if (!grid_x_fits(tg, 256)) return TCFP_ERR_SHAPE;
    split_t_bf16_kernel<<<unsigned(tg), 256, 0, st>>>(g, m, n_out, ap);
    if (hipGetLastError() != hipSuccess) return TCFP_ERR_HIP;
  }
  return wgrad_chunked(ap, m, n_out, x, x_fmt, e_x, k_in, shift, dw,
                       ws + align256(size_t(n_out) * size_t(2 * m) * 2), st);
}

extern "C" size_t tcfp_block_wgrad_presplit_workspace_bytes(int64_t m, int64_t n_out,
                                                           int64_t k_in, int split_lo) {
  if (m < 0 || n_out < 0 || k_in < 0) return 0;
  return wgrad_ws_bytes(m, n_out, k_in, split_lo != 0);
}

extern "C" int tcfp_block_wgrad_presplit(const uint16_t* g_split_t, int split_lo, int64_t m,
                                         int64_t n_out, const uint8_t* x, int x_fmt,
                                         const int8_t* e_x, int64_t k_in, int block, float* dw,
                                         void* workspace, size_t workspace_bytes, void* stream) {
  if (m < 0 || n_out < 0 || k_in < 0 || n_out > INT32_MAX || k_in > INT32_MAX ||
      4 * m > INT32_MAX)
    return TCFP_ERR_SHAPE;
  if (block != 32 && block != 64 && block != 128) return TCFP_ERR_SHAPE;
  if (k_in % block != 0 || m % 4 != 0) return TCFP_ERR_SHAPE;
  // (the single pass contracts over whole 128-byte stages)
  if (split_lo != 1 && (split_lo != 0 || m % 64 != 0)) return TCFP_ERR_SHAPE;
  if (x_fmt != TCFP_FP8_E4M3 && x_fmt != TCFP_FP8_E5M2) return TCFP_ERR_DTYPE;
  if (!g_split_t || !x || !e_x || !dw) return TCFP_ERR_SHAPE;
  if (n_out == 0 || k_in == 0) return TCFP_OK;
  if (!workspace ||
      workspace_bytes < tcfp_block_wgrad_presplit_workspace_bytes(m, n_out, k_in, split_lo))
    return TCFP_ERR_WORKSPACE;
  if (!al16(workspace) || !al16(dw) || !al16(g_split_t)) return TCFP_ERR_ALIGN;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int shift = block == 32 ? 5 : (block == 64 ? 6 : 7);
  return wgrad_chunked(g_split_t, m, n_out, x, x_fmt, e_x, k_in, shift, dw,
                       static_cast<uint8_t*>(workspace), st, split_lo != 0);
}
