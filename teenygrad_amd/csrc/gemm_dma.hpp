// LDS-DMA pipelined MFMA GEMM, two instantiations:
//
//   256 x 256 tiles, one workgroup per CU, for problems that fill the chip
//   with them (the W8A16 linears, big implicit-GEMM convs);
//   128 x 128 tiles, two workgroups per CU, for the deep implicit-GEMM convs
//   with small spatial extent (few, long k-loops).
//
// Same contract as gemm_mfma_kernel (gemm_core.hpp):
//
//   C[m, n] = act( scale[n] * sum_k A[m, k] * B[n, k] + bias[n] )
//
// with A bf16 (plain rows or the NHWC implicit-GEMM gather, C_IN % 8 == 0)
// and B bf16 or int8 [N][K], including the split-K partial output.
//
// Why a second kernel family: the register-staged kernel's loads are
// conditional (bounds, padding), so the compiler waits for all of them
// (vmcnt(0)) before each k-tile's LDS store, and every k-tile pays the full
// global-memory latency.  Here:
//
//  * global -> LDS moves by LDS-DMA (global_load_lds_dwordx4, no staging
//    registers), issued from inline asm so the compiler neither counts it
//    nor waits on it before LDS reads of other stages.  Every k-tile issues
//    the same DMA count (out-of-range chunks read a zero block), so an
//    explicit s_waitcnt vmcnt leaves the newer tiles in flight: NST LDS
//    stages, the DMA NST-1 k-tiles ahead, one barrier per k-tile.
//  * waves are 2 x 2 over the tile; a k-tile (BK = 32, two MFMA k-steps) is
//    2 MB NB fenced bundles, each one MFMA plus a share of the other work:
//    the DMA of k-tile kt+NST-1, LDS reads that refill the one fragment set
//    in place ahead of use (k-tile kt+1's data is complete and published
//    once tile kt starts), and the int8 -> bf16 weight conversion.
//  * 256 x 256: each wave owns 128 x 128 (16 MFMAs per k-step from 8
//    fragments: 0.5 KiB of LDS reads per MFMA, against 1 KiB for 64 x 64
//    wave tiles, which is the CU's LDS bandwidth at the MFMA rate); its 256
//    accumulators per lane live in AGPRs, one wave per SIMD.
//  * int8 weights stay int8 in LDS (half the DMA and LDS bytes) and become
//    bf16 in registers (exact: |q| <= 128 fits bf16's significand); the
//    per-channel scale is applied to the fp32 accumulator.
//
// LDS rows are dense with XOR-swizzled 16-byte chunks so that every
// fragment read (16 consecutive rows per quarter-wave) is bank-conflict
// free.  The k order inside a 32-wide k-tile is permuted identically for
// both operands (k-step st, lane half g reads k = 16 g + 8 st .. + 7), which
// lets one 16-byte read of an int8 row serve both k-steps.
#pragma once

#include "gemm_core.hpp"

namespace teeny {


constexpr int kDmaBK = 32;

template <int BM, int BN, bool INT8B>
constexpr int dma_stage_bytes() {
  return BM * kDmaBK * 2 + BN * kDmaBK * (INT8B ? 1 : 2);
}
template <int BM, int BN, int NST, bool INT8B>
constexpr int dma_lds_bytes() {
  // pipeline stages, or the bf16 C tile of the epilogue, whichever is larger
  return NST * dma_stage_bytes<BM, BN, INT8B>() > BM * (BN + 8) * 2 ? NST * dma_stage_bytes<BM, BN, INT8B>()
                                                                    : BM * (BN + 8) * 2;
}

// BM x BN tile, NST LDS stages, MINW workgroups per CU; SPLIT: split-K
// partial output when p.ws is set (a separate instantiation: the partial
// store path alone costs the 256 x 256 tile spills).  WAVES_N: the four
// waves as 2 x 2 blocks of the tile, or 1 x 4 (each wave all BM rows and a
// quarter of the columns: with int8 weights every weight fragment is then
// converted by one wave only, half the VALU work of the 2 x 2 layout, whose
// two waves of a column block both convert it).
template <int BM, int BN, int NST, int MINW, bool INT8B, int AMODE, bool SPLIT, int WAVES_N = 2>
__global__ __launch_bounds__(256, MINW) void gemm_dma_kernel(GemmParams p) {
  constexpr int BK = kDmaBK;
  constexpr int WAVES_M = 4 / WAVES_N;
  constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;  // wave block
  constexpr int MB = WM / 32, NB = WN / 32;            // 32 x 32 MFMA blocks per wave
  constexpr int H = MB * NB;                           // MFMA bundles per k-step
  constexpr int A_BYTES = BM * BK * 2;
  constexpr int B_BYTES = BN * BK * (INT8B ? 1 : 2);
  constexpr int STAGE = A_BYTES + B_BYTES;
  constexpr int A_LD = A_BYTES / 16 / 256;             // DMA rounds per k-tile (A)
  constexpr int B_LD = B_BYTES / 16 / 256;             // DMA rounds per k-tile (B)
  constexpr int DMA_PER_KT = A_LD + B_LD;
  // k-tiles whose DMA may still fly at the end of a k-tile (kt+3 .. kt+NST-1)
  constexpr int INFLIGHT = DMA_PER_KT * (NST - 3);
  static_assert(AMODE == kAPlain || AMODE == kAConvVec, "16-byte gather only");
  static_assert(A_BYTES % 4096 == 0 && B_BYTES % 4096 == 0, "whole DMA rounds per k-tile");
  static_assert(MB >= 2 && NB >= 2 && MB + NB <= H && DMA_PER_KT <= 2 * H, "bundle schedule");
  static_assert(NST >= 4 && INFLIGHT < 16, "stages / vmcnt field");
  extern __shared__ __attribute__((aligned(16))) char smem[];

  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6, g = lane >> 5, c = lane & 31;
  const int wm = w / WAVES_N, wn = w % WAVES_N;  // wave block: rows wm*WM.. of m, wn*WN.. of n

  const int tiles_m = (p.M + BM - 1) / BM;
  const int tiles_n = (p.N + BN - 1) / BN;
  const int n_tiles = tiles_m * tiles_n;
  const int id = xcd_remap(blockIdx.x, gridDim.x);
  const int tile = id % n_tiles;
  const int split = id / n_tiles;  // 0 unless split-K
  // consecutive tiles (one XCD's run) share the larger operand (p.n_fast)
  const bool n_fast = p.n_fast != 0;
  int tm = n_fast ? tile / tiles_n : tile % tiles_m;
  int tn = n_fast ? tile % tiles_n : tile / tiles_m;
  if (p.group > 0) {
    // slow dimension s (M when n_fast) in groups of p.group tiles; inside a
    // group s varies fastest, then the other dimension
    const int ts = n_fast ? tiles_m : tiles_n, tf = n_fast ? tiles_n : tiles_m;
    const int g0 = tile / (p.group * tf) * p.group;
    const int gsz = min(p.group, ts - g0);
    const int r = tile - g0 * tf;
    const int s_idx = g0 + r % gsz, f_idx = r / gsz;
    tm = n_fast ? s_idx : f_idx;
    tn = n_fast ? f_idx : s_idx;
  }
  const int m0 = tm * BM;
  const int n0 = tn * BN;
  const int n_k_all = (p.K + BK - 1) / BK;
  const bool split_k = SPLIT && p.ws != nullptr;
  const int kt_begin = split_k ? split * p.kt_split : 0;
  const int n_k = (split_k ? min(n_k_all, kt_begin + p.kt_split) : n_k_all) - kt_begin;
  const int k_first = kt_begin * BK;

  // ── DMA mapping.  A / bf16 B stage: 1024 slots of 16 B; slot t + 256 i is
  // row t / 4 + 64 i at chunk position t % 4 and holds data chunk
  // (t % 4) ^ ((t >> 4) & 3) (the row's swizzle, independent of i).
  // int8 B stage: 512 slots; slot t + 256 i is row t / 2 + 128 i at position
  // t % 2, data chunk (t % 2) ^ ((t >> 4) & 1).
  const int a_row0 = tid >> 2;
  const int a_col = ((tid & 3) ^ ((tid >> 4) & 3)) * 8;           // k offset (elements)
  const int b_row0 = INT8B ? (tid >> 1) : (tid >> 2);
  const int b_col = INT8B ? ((tid & 1) ^ ((tid >> 4) & 1)) * 16   // k offset (int8 elements)
                          : a_col;
  constexpr int B_RSTEP = INT8B ? 128 : 64;

  // Sources are buffer offsets (bytes): rows past M / N read the last valid
  // row (their products only reach discarded outputs) and a chunk that must
  // read as zero (k past K, a padding tap, k-tiles past the end) gets an
  // offset past the buffer extent, which the hardware returns as zeros.
  const __amdgpu_buffer_rsrc_t a_rsrc = buffer_rsrc(p.A, p.a_bytes);
  const __amdgpu_buffer_rsrc_t b_rsrc = buffer_rsrc(p.B, p.b_bytes);
  int a_off[A_LD];  // plain: row start; conv: tap (0, 0), channel 0 of the row's window
  int a_ih0[A_LD], a_iw0[A_LD];
#pragma unroll
  for (int i = 0; i < A_LD; ++i) {
    const int m = min(m0 + a_row0 + 64 * i, p.M - 1);
    if constexpr (AMODE == kAPlain) {
      a_off[i] = static_cast<int>(static_cast<int64_t>(m) * p.lda * 2);
      a_ih0[i] = a_iw0[i] = 0;
    } else {
      const int ow = m % p.OW;
      const int t = m / p.OW;
      const int oh = t % p.OH;
      const int b = t / p.OH;
      a_ih0[i] = oh * p.SH - p.PH;
      a_iw0[i] = ow * p.SW - p.PW;
      a_off[i] = static_cast<int>(
          2 * (static_cast<int64_t>(b) * p.H * p.W * p.Cin + static_cast<int64_t>(a_ih0[i] * p.W + a_iw0[i]) * p.Cin));
    }
  }
  int b_off[B_LD];
#pragma unroll
  for (int i = 0; i < B_LD; ++i) {
    const int n = min(n0 + b_row0 + B_RSTEP * i, p.N - 1);
    b_off[i] = static_cast<int>(static_cast<int64_t>(n) * p.ldb * (INT8B ? 1 : 2));
  }
  // Implicit-GEMM k decomposition, stepped per k-tile: tap (kh, kw), channel
  // ci and the byte offset 2 ((kh W + kw) C_IN + ci).  When C_IN % BK == 0 a
  // k-tile never straddles a tap and the state of its first column is
  // wave-uniform (scalar registers); otherwise each thread steps its own.
  const bool tap_uniform = AMODE == kAConvVec && p.Cin % BK == 0;
  struct TapState {
    int ci, kw, kh, off;
  };
  auto tap_at = [&](int k) {
    TapState t;
    t.ci = k % p.Cin;
    const int r = k / p.Cin;
    t.kw = r % p.KW;
    t.kh = r / p.KW;
    t.off = 2 * ((t.kh * p.W + t.kw) * p.Cin + t.ci);
    return t;
  };
  TapState u_tap{0, 0, 0, 0}, v_tap{0, 0, 0, 0};
  if constexpr (AMODE == kAConvVec) {
    if (tap_uniform) u_tap = tap_at(k_first);
    else v_tap = tap_at(k_first + a_col);
  }
  auto tap_step = [&](TapState &t, bool once) __attribute__((always_inline)) {
    t.ci += BK;
    t.off += 2 * BK;
    while (t.ci >= p.Cin) {
      t.ci -= p.Cin;
      if (++t.kw == p.KW) {
        t.kw = 0;
        ++t.kh;
        t.off += 2 * (p.W - p.KW) * p.Cin;
      }
      if (once) break;
    }
  };
  const uint32_t lds0 = lds_address(smem);
  // DMA instruction d (0 .. DMA_PER_KT-1) of k-tile kt into stage kt % NST
  // (zeros past n_k): d < A_LD are activation rounds, the rest weight rounds.
  // The activation gather of a conv needs (kh, kw, ci) for k-tile kt:
  // advance_k() steps it once the k-tile's A rounds are out.
  auto dma_one = [&](int kt, int d) __attribute__((always_inline)) {
    const uint32_t st_base = lds0 + (kt % NST) * STAGE;
    const int k0 = k_first + kt * BK;
    const bool live = kt < n_k;
    if (d < A_LD) {
      const int i = d;
      const int k = k0 + a_col;
      int off;
      if constexpr (AMODE == kAPlain) {
        off = (live & (k < p.K)) ? a_off[i] + 2 * k : kOffNone;
      } else {
        auto gather = [&](const TapState &t, int col_bytes) __attribute__((always_inline)) {
          const int ih = a_ih0[i] + t.kh, iw = a_iw0[i] + t.kw;
          const bool ok = live & (k < p.K) & (static_cast<unsigned>(ih) < static_cast<unsigned>(p.H)) &
                          (static_cast<unsigned>(iw) < static_cast<unsigned>(p.W));
          return ok ? a_off[i] + t.off + col_bytes : kOffNone;
        };
        off = tap_uniform ? gather(u_tap, 2 * a_col) : gather(v_tap, 0);
      }
      buffer_lds_dma16(a_rsrc, off, __builtin_amdgcn_readfirstlane(st_base + i * 4096 + w * 1024));
    } else {
      const int i = d - A_LD;
      const int k = k0 + b_col;
      const int off = (live & (k < p.K)) ? b_off[i] + k * (INT8B ? 1 : 2) : kOffNone;
      buffer_lds_dma16(b_rsrc, off, __builtin_amdgcn_readfirstlane(st_base + A_BYTES + i * 4096 + w * 1024));
    }
  };
  auto advance_k = [&]() __attribute__((always_inline)) {
    if constexpr (AMODE == kAConvVec) {
      if (tap_uniform) tap_step(u_tap, true);
      else tap_step(v_tap, false);
    }
  };
  auto dma_tile = [&](int kt) __attribute__((always_inline)) {
#pragma unroll
    for (int d = 0; d < DMA_PER_KT; ++d) {
      dma_one(kt, d);
      if (d == A_LD - 1) advance_k();
    }
  };

  // ── fragment offsets (bytes within a stage).  Activations (B operand):
  // block j row wm*WM + 32 j + c, chunk 2 g + st at position
  // chunk ^ ((row >> 2) & 3) = chunk ^ ((c >> 2) & 3).  bf16 weights (A
  // operand) likewise with wn.  int8 weights: row wn*WN + 32 i + c, chunk g
  // at position g ^ ((c >> 3) & 1), 16 bytes = both k-steps.
  const int sw_a = (c >> 2) & 3;
  const int x_off = (wm * WM + c) * 64;
  const int w_off = INT8B ? A_BYTES + (wn * WN + c) * 32 + ((g ^ ((c >> 3) & 1)) << 4)
                          : A_BYTES + (wn * WN + c) * 64;

  f32x16 acc[NB][MB];
#pragma unroll
  for (int i = 0; i < NB; ++i)
#pragma unroll
    for (int j = 0; j < MB; ++j) acc[i][j] = zero16();

  // A fragment set holds one k-tile: x[st][j] activations, w[st][i] bf16
  // weights (for int8, the converted weights).
  typedef bf16x8 frag_t;
  struct FragSet {
    frag_t x[2][MB];
    frag_t w[2][NB];
  };
  auto read_x = [&](const char *st_ptr, int st, int j, FragSet &f) __attribute__((always_inline)) {
    f.x[st][j] = *reinterpret_cast<const frag_t *>(st_ptr + x_off + j * 32 * 64 + (((2 * g + st) ^ sw_a) << 4));
  };
  auto read_w = [&](const char *st_ptr, int st, int i, FragSet &f) __attribute__((always_inline)) {
    f.w[st][i] = *reinterpret_cast<const frag_t *>(st_ptr + w_off + i * 32 * 64 + (((2 * g + st) ^ sw_a) << 4));
  };
  // int8: one 16-byte read per n-block covers both k-steps ...
  auto read_q = [&](const char *st_ptr, int i) __attribute__((always_inline)) {
    return *reinterpret_cast<const u32x4 *>(st_ptr + w_off + i * 32 * 32);
  };
  // ... and half of it (8 weights, one k-step) becomes one bf16 fragment
  auto convert_q = [&](const u32x4 &q, int st, int i, FragSet &f) __attribute__((always_inline)) {
    bf16 e[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int byte = 8 * st + t;
      const int8_t b = static_cast<int8_t>((q[byte >> 2] >> (8 * (byte & 3))) & 0xffu);
      e[t] = static_cast<bf16>(static_cast<float>(b));
    }
    __builtin_memcpy(&f.w[st][i], e, 16);
  };
  // ... or a quarter of it: weights 2r, 2r + 1 of that fragment
  auto convert_q2 = [&](const u32x4 &q, int st, int i, int r, FragSet &f) __attribute__((always_inline)) {
    const int byte = 8 * st + 2 * r;
    const uint32_t word = q[byte >> 2] >> (8 * (byte & 3));
    const bf16x2 pair = cvt_pk_bf16(static_cast<float>(static_cast<int8_t>(word & 0xffu)),
                                    static_cast<float>(static_cast<int8_t>((word >> 8) & 0xffu)));
    f.w[st][i][2 * r] = pair[0];
    f.w[st][i][2 * r + 1] = pair[1];
  };
  // One k-tile as 2H fenced bundles.  Bundle b issues MFMA (st, i, j) =
  // (b / H, (b % H) / MB, b % MB) plus a share of the other work: the DMA of
  // k-tile kt+NST-1 (first bundles) and LDS reads that refill the single
  // fragment set in place: during the k-step-0 MFMAs the k-step-1 slots
  // (free since the previous k-tile) receive this k-tile's k-step-1
  // fragments; during the k-step-1 MFMAs the k-step-0 slots (just freed)
  // receive k-tile kt+1's (complete and published once tile kt starts).
  // int8 weights: one 16-byte read per n-block (q) serves both k-steps; its
  // k-step-1 half is converted during the first half of the k-tile, then q
  // is refilled with k-tile kt+1's chunks, whose k-step-0 half is converted
  // in the second half, after the last k-step-0 MFMA that reads the slot.
  // Bundles of the int8 work (c1: k-step-1 conversion of n-block i; qr: read
  // of k-tile kt+1's chunk i; xr: its k-step-0 activation fragment j; c0: its
  // k-step-0 conversion of n-block i):
  //   H = 16 (256 x 256): each conversion in four quarters (two weights, a
  //            few VALU instructions) spread over the 32 bundles, so that no
  //            bundle's VALU work outlasts its MFMA: c1 quarter r at 4i + r,
  //            qr = 4i + 4, xr = 20 + j, c0 quarter r at 16 + 4i + r
  //   H = 8  (256 x 128): c1 = 4 + i,  qr = 8 + i,  xr = 10 + j, c0 = 14 + i
  //   H = 4  (128 x 128): c1 = i,      qr = 2 + i,  xr = 4 + j,  c0 = 6 + i
  // (c1 before the first k-step-1 MFMA of block i at H + MB i; qr after c1;
  // xr after the last k-step-0 MFMA reading slot j, (NB - 1) MB + j; c0
  // after the last one reading block i, MB i + MB - 1.)
  // The bundle -> block maps are plain index arithmetic on the (unrolled)
  // bundle number, so every fragment index is a compile-time constant
  // (a run-time index would put the fragment set in scratch memory).
  //   H = 16, MB = 8, NB = 2 (256 x 256, waves 1 x 4): c1 quarter r of block
  //            i at 8 i + 2 r + 1, qr = 8 + 8 i, xr = 16 + j, c0 quarters at
  //            10 + 2 r (block 0) and 24 + 2 r (block 1)
  static_assert((H == 16 && ((MB == 4 && NB == 4) || (MB == 8 && NB == 2))) || (H == 8 && MB == 4 && NB == 2) ||
                    (H == 4 && MB == 2 && NB == 2),
                "int8 schedule covers H = 4, 8, 16");
  constexpr int kC1 = H == 16 ? 4 : H == 8 ? 4 : 0, kC1Step = H == 16 ? 2 : 1;
  constexpr int kQr = H == 16 ? 16 : H == 8 ? 8 : 2;
  constexpr int kXr = H == 16 ? 20 : H == 8 ? 10 : 4;
  constexpr int kC0 = H == 16 ? 24 : H == 8 ? 14 : 6, kC0Step = H == 16 ? 2 : 1;
  // The reads of k-tile kt+1 are issued unconditionally: on the last k-tile
  // they read stage (kt+1) % NST, whose zero-source DMA completed with the
  // same wait as a live tile's, and the fragments are never used.  A branch
  // around them would split the bundles and make the compiler's LDS waits
  // assume the path without the reads (each read then waited on at once).
  FragSet f;
  u32x4 q[NB];
  auto ktile = [&](int kt) __attribute__((always_inline)) {
    const char *cu = smem + (kt % NST) * STAGE;
    const char *nx = smem + ((kt + 1) % NST) * STAGE;
    constexpr bool more = true;
#pragma unroll
    for (int b = 0; b < 2 * H; ++b) {
      const int st = b / H, i = (b % H) / MB, j = b % MB;
      if (b < DMA_PER_KT) {
        dma_one(kt + NST - 1, b);
        if (b == A_LD - 1) advance_k();
      }
      if constexpr (INT8B && H == 16 && MB == 8) {
        if (b < MB) read_x(cu, 1, b, f);  // this k-tile's k-step 1
        // k-step-1 conversions: block 0 at b = 1, 3, 5, 7, block 1 at 9 .. 15
        // (first k-step-1 MFMAs of the blocks at b = 16 and 24)
        if (b < 16 && (b & 1)) convert_q2(q[b >> 3], 1, b >> 3, (b >> 1) & 3, f);
        // next k-tile's chunks, each after its block's k-step-1 conversion
        if (more && b == 8) q[0] = read_q(nx, 0);
        if (more && b == 16) q[1] = read_q(nx, 1);
        // next k-tile's k-step-0 activations: slot j was last read at b = 8 + j
        if (more && b >= 16 && b < 24) read_x(nx, 0, b - 16, f);
        // next k-tile's k-step-0 conversions, after the last k-step-0 MFMA of
        // the block (b = 7, 15) and its chunk read
        if (more && b >= 10 && b <= 16 && !(b & 1)) convert_q2(q[0], 0, 0, (b - 10) >> 1, f);
        if (more && b >= 24 && !(b & 1)) convert_q2(q[1], 0, 1, (b - 24) >> 1, f);
      } else if constexpr (INT8B && H == 16) {
        if (b < MB) read_x(cu, 1, b, f);  // this k-tile's k-step 1
        if (b < 16) convert_q2(q[b >> 2], 1, b >> 2, b & 3, f);
        if (more && b >= 4 && b <= 16 && (b & 3) == 0) q[(b >> 2) - 1] = read_q(nx, (b >> 2) - 1);
        if (more && b >= 20 && b < 24) read_x(nx, 0, b - 20, f);
        if (more && b >= 16) convert_q2(q[(b - 16) >> 2], 0, (b - 16) >> 2, b & 3, f);
      } else if constexpr (INT8B) {
        if (b < MB) read_x(cu, 1, b, f);  // this k-tile's k-step 1
        if (b >= kC1 && b < kC1 + kC1Step * NB && (b - kC1) % kC1Step == 0)
          convert_q(q[(b - kC1) / kC1Step], 1, (b - kC1) / kC1Step, f);
        if (more && b >= kQr && b < kQr + NB) q[b - kQr] = read_q(nx, b - kQr);
        if (more && b >= kXr && b < kXr + MB) read_x(nx, 0, b - kXr, f);
        if (more && b >= kC0 && b < kC0 + kC0Step * NB && (b - kC0) % kC0Step == 0)
          convert_q(q[(b - kC0) / kC0Step], 0, (b - kC0) / kC0Step, f);
      } else {
        if (b < H) {
          // this k-tile's k-step 1: MB activation and NB weight reads
          if (b < MB) read_x(cu, 1, b, f);
          else if (b < MB + NB) read_w(cu, 1, b - MB, f);
        } else if (more) {
          // next k-tile's k-step 0
          const int r = b - H;
          if (r < MB) read_x(nx, 0, r, f);
          else if (r < MB + NB) read_w(nx, 0, r - MB, f);
        }
      }
      acc[i][j] = mfma32x32x16(f.w[st][i], f.x[st][j], acc[i][j]);
      __builtin_amdgcn_sched_barrier(0);
    }
    // DMA of k-tiles <= kt+2 complete (newer ones may still fly), then the
    // barrier that publishes them
    __builtin_amdgcn_s_waitcnt(0xF70 | INFLIGHT);
    __syncthreads();
  };

  // prologue: k-tiles 0 .. NST-2 in flight, 0 and 1 complete and published;
  // k-step 0 of k-tile 0 into the fragment set (int8: with its chunks in q)
#pragma unroll
  for (int t = 0; t < NST - 1; ++t) dma_tile(t);
  __builtin_amdgcn_s_waitcnt(0xF70 | INFLIGHT);
  __syncthreads();
#pragma unroll
  for (int j = 0; j < MB; ++j) read_x(smem, 0, j, f);
  if constexpr (INT8B) {
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      q[i] = read_q(smem, i);
      convert_q(q[i], 0, i, f);
    }
  } else {
#pragma unroll
    for (int i = 0; i < NB; ++i) read_w(smem, 0, i, f);
  }
  for (int kt = 0; kt < n_k; ++kt) ktile(kt);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // trailing zero-source DMA
  __syncthreads();

  if (split_k) {
    // split-K partial: raw fp32 accumulators, four consecutive n per lane
    float *wsp = p.ws + static_cast<int64_t>(split) * p.M * p.N;
#pragma clang loop unroll(full)
    for (int j = 0; j < MB; ++j) {
      const int m = m0 + wm * WM + j * 32 + c;
#pragma clang loop unroll(full)
      for (int i = 0; i < NB; ++i) {
#pragma clang loop unroll(full)
        for (int v4 = 0; v4 < 4; ++v4) {
          const int n = n0 + wn * WN + i * 32 + 8 * v4 + 4 * g;
          if (m < p.M && n < p.N) {
            float *dst = wsp + static_cast<int64_t>(m) * p.N + n;
            if (n + 4 <= p.N && (p.N & 3) == 0) {
              f32x4 v{acc[i][j][4 * v4], acc[i][j][4 * v4 + 1], acc[i][j][4 * v4 + 2], acc[i][j][4 * v4 + 3]};
              *reinterpret_cast<f32x4 *>(dst) = v;
            } else {
              for (int e = 0; e < 4 && n + e < p.N; ++e) dst[e] = acc[i][j][4 * v4 + e];
            }
          }
        }
      }
    }
    return;
  }

  // ── epilogue: scale / bias / activation, bf16 C tile through LDS, 16-byte
  // row chunks out (coalesced).
  constexpr int CP = BN + 8;
  bf16 *cs = reinterpret_cast<bf16 *>(smem);
  // scale / bias per group of four columns (shared by the MB row blocks)
#pragma clang loop unroll(full)
  for (int i = 0; i < NB; ++i)
#pragma clang loop unroll(full)
    for (int v4 = 0; v4 < 4; ++v4) {
      float mul[4], add[4];
      epi_coeffs(p, n0 + wn * WN + i * 32 + 8 * v4 + 4 * g, mul, add);
#pragma clang loop unroll(full)
      for (int j = 0; j < MB; ++j)
#pragma clang loop unroll(full)
        for (int e = 0; e < 4; ++e) acc[i][j][4 * v4 + e] = __builtin_fmaf(acc[i][j][4 * v4 + e], mul[e], add[e]);
    }
  const EpiAct ea = epi_act(p.act);
  if (ea.sig) {
#pragma clang loop unroll(full)
    for (int i = 0; i < NB; ++i)
#pragma clang loop unroll(full)
      for (int j = 0; j < MB; ++j)
#pragma clang loop unroll(full)
        for (int v = 0; v < 16; ++v) acc[i][j][v] = epi_sig(acc[i][j][v], ea);
  }
  const float lo = ea.relu ? 0.0f : -INFINITY;
#pragma clang loop unroll(full)
  for (int j = 0; j < MB; ++j) {
    const int ml = wm * WM + j * 32 + c;
#pragma clang loop unroll(full)
    for (int i = 0; i < NB; ++i) {
#pragma clang loop unroll(full)
      for (int v4 = 0; v4 < 4; ++v4) {
        const int nl = wn * WN + i * 32 + 8 * v4 + 4 * g;
        bf16x4 o4;
#pragma clang loop unroll(full)
        for (int e = 0; e < 4; ++e) {
          const float r = acc[i][j][4 * v4 + e];
          o4[e] = static_cast<bf16>(r < lo ? lo : r);
        }
        // 16-byte chunk nl / 8 of row ml sits at chunk (nl / 8) ^ ((ml >> 4) & 1):
        // rows c and c + 16 of one write instruction then use different banks
        *reinterpret_cast<bf16x4 *>(cs + ml * CP + (((nl >> 3) ^ ((ml >> 4) & 1)) << 3) + (nl & 7)) = o4;
      }
    }
  }
  __syncthreads();
  constexpr int CPR_C = BN / 8;       // 16-byte chunks per C row
  constexpr int RPP_C = 256 / CPR_C;  // rows per pass
  const bool vec16 = (p.ldc % 8 == 0) && ((reinterpret_cast<uintptr_t>(p.C) & 15) == 0);
#pragma clang loop unroll(full)
  for (int r0 = 0; r0 < BM; r0 += RPP_C) {
    const int ml = r0 + tid / CPR_C, nl = (tid % CPR_C) * 8;
    const int m = m0 + ml, n = n0 + nl;
    if (m < p.M && n < p.N) {
      const u32x4 v = *reinterpret_cast<const u32x4 *>(cs + ml * CP + (((nl >> 3) ^ ((ml >> 4) & 1)) << 3));
      bf16 *dst = p.C + static_cast<int64_t>(m) * p.ldc + n;
      if (vec16 && n + 8 <= p.N) {
        // non-temporal: the output does not displace the operand k-slices
        // the XCD's other tiles still read (11008 -> 4096 316 -> 311 us)
        __builtin_nontemporal_store(v, reinterpret_cast<u32x4 *>(dst));
      } else {
        bf16 e[8];
        __builtin_memcpy(e, &v, 16);
        for (int t = 0; t < 8 && n + t < p.N; ++t) dst[t] = e[t];
      }
    }
  }
}

// Whether the LDS-DMA kernels can take this problem: 16-byte chunks must
// never straddle a row or K (bf16: K % 8, int8: K % 16, 16-byte aligned
// operands and leading dimensions) and the gather must be the vector one.
template <bool INT8B, int AMODE>
inline bool dma_gemm_ok(const GemmParams &p) {
  if (AMODE != kAPlain && AMODE != kAConvVec) return false;
  if (p.K % (INT8B ? 16 : 8) != 0) return false;
  if (!aligned(p.A, 16) || !aligned(p.B, 16)) return false;
  if (AMODE == kAPlain && p.lda % 8 != 0) return false;
  return p.ldb % (INT8B ? 16 : 8) == 0;
}

// The 256 x 256 kernel: N must fill a 256-wide tile, the k-loop must be
// long enough (K >= 512) for the pipeline to outweigh the 256 x 256
// epilogue, and 256 x 256 tiles must still give every CU a workgroup.
template <bool INT8B, int AMODE>
inline bool big_gemm_fits(const GemmParams &p) {
  return dma_gemm_ok<INT8B, AMODE>(p) && p.K >= 16 * kDmaBK && p.N >= 256 &&
         tiles_of(p, 256, 256) >= device_cu_count();
}

template <int BM, int BN, int NST, int MINW, bool INT8B, int AMODE, bool SPLIT, int WAVES_N = 2>
inline void launch_dma_gemm(const GemmParams &p, hipStream_t s, int splits = 1) {
  constexpr int bytes = dma_lds_bytes<BM, BN, NST, INT8B>();
  static const bool attr_set = [] {
    return hipFuncSetAttribute(
               reinterpret_cast<const void *>(&gemm_dma_kernel<BM, BN, NST, MINW, INT8B, AMODE, SPLIT, WAVES_N>),
               hipFuncAttributeMaxDynamicSharedMemorySize, bytes) == hipSuccess;
  }();
  (void)attr_set;
  const int grid = static_cast<int>(tiles_of(p, BM, BN)) * (SPLIT ? splits : 1);
  hipLaunchKernelGGL((gemm_dma_kernel<BM, BN, NST, MINW, INT8B, AMODE, SPLIT, WAVES_N>), dim3(grid), dim3(256),
                     bytes, s, p);
}

// The 256 x 256 kernel walks its tiles in groups of 8 along the slow
// dimension: the 32 tiles an XCD runs at a time form an 8 x 4 block, whose
// operand k-slices its L2 then serves several times (measured on the W8A16
// shapes: 4096 -> 11008 425 -> 350 us, 11008 -> 4096 323 -> 317 us).
// int8 weights take the 1 x 4 wave layout (each weight converted once per
// workgroup): 4096 -> 11008 355 -> 345 us, 11008 -> 4096 327 -> 316 us,
// interleaved on one box; bf16 weights keep 2 x 2 (fewer LDS bytes per MFMA).
template <bool INT8B, int AMODE>
inline void launch_big_gemm(GemmParams p, hipStream_t s) {
  p.group = 8;
  if constexpr (INT8B) launch_dma_gemm<256, 256, 4, 1, INT8B, AMODE, false, 4>(p, s);
  else launch_dma_gemm<256, 256, 4, 1, INT8B, AMODE, false>(p, s);
}

}  // namespace teeny
