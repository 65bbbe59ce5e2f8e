// Band-tiled convolution with streamed weights, for NHWC convs whose input
// rows are short (built for the 14x14 3x3 ResNet layers; the template also
// takes 28-wide outputs, 7x7 outputs two images at a time, stride-2 3x3 convs
// to 7x7 outputs, the stride-2 dx mode below, and int8 weights), here for
// stride 1:
//
//   y[b, oh, ow, n] = act( scale[n] * sum_{kh, kw, ci} x[b, oh - PH + kh, ow - PW + kw, ci]
//                                      * w[n, kh, kw, ci] + bias[n] )
//
// with w bf16, or int8 whose per-channel scale multiplies the accumulator
// (teeny-quant's dequantize_affine, affine.rs:151-161, applied in the
// epilogue; the int8 values become bf16 in registers, exactly).
//
// The implicit GEMM reads every input pixel once per tap (9x for a 3x3)
// from L2.  Here a workgroup owns RB whole output rows of one image (RB * OW
// = 196 pixels: a 14x14 image, or 7 rows of a 28x28 one) and BN output
// channels; per 32-channel chunk of C_IN, one LDS-DMA pass brings the rows'
// input with its halo, (RB + KH - 1) x (OW + KW - 1) pixels (padding read as
// zeros through out-of-extent buffer offsets), and the chunk's BN x KH x KW
// x 32 weights; all taps are then read from LDS.  Three LDS stages where
// they fit (the DMA of the chunk after next is issued before the current
// chunk's MFMAs), else two.
//
// One wave per 32 pixels of the band (seven for 196 pixels), or two (eight
// for the 98 of two 7x7 images, each taking one of the two k-steps of every
// tap, their sums added through LDS at the unit's end); wave w owns pixels
// 32 w .. 32 w + 31 (the last wave's pixels past the band read the last
// pixel's window and are not stored) and all BN channels: per k-step (16
// channels of one tap) one pixel
// fragment and BN / 32 weight fragments feed BN / 32
// v_mfma_f32_32x32x16_bf16 computing D[n][px].  LDS rows: weight rows of
// KH*KW 64-byte (bf16) or 32-byte (int8) tap segments plus one 16-byte pad
// slot (an odd number of 16-byte units per row: conflict-free fragment
// reads of consecutive rows); halo pixels of 4 x 16 bytes with chunk q of
// halo slot cs (the halo column, or its phase-plane slot at stride 2) at
// position q ^ ((cs >> 2) & 3).  Units (band, channel tile) are dealt to
// workgroups XCD by XCD, so the channel tiles of a band read its input rows
// from one L2.  Epilogue through a
// per-wave 4 KiB LDS slice of the stage buffer the unit's last chunk used
// (after a barrier), 64 channels at a time, written back as whole
// 128-byte segments of the pixels' rows; the vmcnt waits count the
// epilogue's stores (operations retire in issue order), so they stay in
// flight.
#pragma once

#include <type_traits>

#include "gemm_core.hpp"

namespace teeny {

struct TileConvParams {
  const bf16 *x;     // [B, H, W, C_IN]
  const void *w;     // [C_OUT, KH, KW, C_IN], bf16 or int8
  const float *scale, *bias;
  const bf16 *bias_bf16;
  bf16 *y;           // [B, OH, OW, C_OUT]
  int B, H, W, Cin, Cout, OH, PH, PW, act;
  int x_bytes, w_bytes;  // byte extents (below 2^31)
  // stride-2 3x3 dx mode: element offset of each sub-pixel phase's weights
  int phase_off[4];
};

// IPB > 1: a band is IPB whole images of RB = OH rows (the 7x7 layers),
// their halos stacked (image i's halo rows at i (RB + KH - 1)).
// S2: stride 2 (3x3): the halo holds input rows 2 oh0 - PH .. 2 (oh0 + RB -
// 1) - PH + 2 and, per row, its columns as two phase planes, the even halo
// columns hc = 2 j at slots j = 0 .. OWT, then the odd ones at OWT + 1 + j,
// so the 32 consecutive output pixels of a fragment read consecutive slots.
// KS = 2: two waves per 32-pixel block, each taking one of the two k-steps
// of every tap (16 of a chunk's 32 channels); their sums meet in LDS at the
// unit's end.  For bands of few pixels (four blocks), so that each SIMD runs
// two waves.
template <int KH, int KW, int OWT, int RB, int BN, bool INT8B, bool DX2 = false, int IPB = 1, bool S2 = false,
          int KS = 1>
struct TileShape {
  static constexpr int NPX = RB * OWT * IPB;     // pixels per band
  static constexpr int NPB = (NPX + 31) / 32;    // 32-pixel blocks
  static constexpr int NW = NPB * KS;            // waves
  static constexpr int NT = 64 * NW;
  static constexpr int PLANE = OWT + 1;          // stride 2: slots per column phase plane
  // dx mode: a phase reads dy rows u, u + 1 and columns v, v + 1 (no padding)
  static constexpr int HRI = DX2 ? RB + 1 : (S2 ? 2 * RB + 1 : RB + KH - 1);  // halo rows per image of the band
  static constexpr int HR = HRI * IPB, HC = DX2 ? OWT + 1 : (S2 ? 2 * PLANE : OWT + KW - 1);
  static_assert(IPB == 1 || !DX2, "multi-image bands: forward only");
  static_assert(!S2 || (KH == 3 && KW == 3 && !DX2), "stride-2 mode: 3x3 forward");
  static constexpr int HSLOTS = HR * HC * 4;     // 16-byte halo slots (32 channels per pixel)
  static constexpr int QT = INT8B ? 2 : 4;       // 16-byte slots per tap segment
  // taps of a unit, at most (dx mode: row phase a = 1 with both column
  // phases, 2 + 4 taps)
  static constexpr int TAPS = DX2 ? 6 : KH * KW;
  static constexpr int RS = TAPS * QT + 1;       // slots per weight row (+ 1 pad slot)
  static constexpr int WSLOTS = BN * RS;
  static constexpr int HINSTR = (HSLOTS + 63) / 64, WINSTR = (WSLOTS + 63) / 64;
  static constexpr int INSTR = HINSTR + WINSTR;  // DMA instructions per stage (workgroup)
  static constexpr int DI = (INSTR + NW - 1) / NW;  // per wave (the excess repeat the first ones)
  static constexpr int HBYTES = HINSTR * 1024, WBYTES = WINSTR * 1024;
  static constexpr int STAGE = HBYTES + WBYTES;
  static constexpr int STG = 4096;               // epilogue slice per wave
  // LDS stages: three (two DMA passes in flight) where they fit, else two
  static constexpr int NSTG = 3 * STAGE + 2 * BN * 4 <= 160 * 1024 ? 3 : 2;
  static constexpr int LDS = NSTG * STAGE + 2 * BN * 4;
  static_assert(NPB * STG + (KS - 1) * NPB * 8192 <= STAGE, "epilogue slices (and k-split sums) fit one stage buffer");
  static_assert(KS == 1 || (KS == 2 && !DX2 && !INT8B), "k-split waves: bf16 forward");
  static_assert(DI * NW - INSTR <= INSTR, "excess DMA instructions repeat real ones");
  static_assert(RS % 2 == 1, "odd number of 16-byte units per weight row");
  static_assert(BN % 64 == 0 && NW <= 16, "tile");
  static_assert(LDS <= 160 * 1024, "LDS");
};

template <int KH, int KW, int OWT, int RB, int BN, bool INT8B, bool DX2 = false, int IPB = 1, bool S2 = false,
          int KS = 1>
__global__ __launch_bounds__((TileShape<KH, KW, OWT, RB, BN, INT8B, DX2, IPB, S2, KS>::NT), 1) void conv_tile_kernel(
    TileConvParams p) {
  using S = TileShape<KH, KW, OWT, RB, BN, INT8B, DX2, IPB, S2, KS>;
  static_assert(!DX2 || (KH == 3 && KW == 3 && !INT8B), "dx mode: bf16 3x3 stride 2 pad 1");
  constexpr int NW = S::NW, HC = S::HC, DI = S::DI, NB = BN / 32;
  constexpr int EPI_STORES = 4 * (BN / 64) * (DX2 ? 2 : 1);  // per unit (dx mode: two phases)
  static_assert((S::NSTG - 2) * DI + 2 * EPI_STORES < 64 && S::NSTG <= 3, "vmcnt field / wait cases");
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int tid = threadIdx.x;
  const int lane = tid & 63, g = lane >> 5, c = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  float *const cmul = reinterpret_cast<float *>(smem + S::NSTG * S::STAGE);
  float *const cadd = cmul + BN;

  const int bands_per_img = p.OH / RB;
  const int n_tiles = p.Cout / BN;
  const int n_bands = IPB > 1 ? (p.B + IPB - 1) / IPB : p.B * bands_per_img;
  const int per_phase = n_bands * n_tiles;
  const int n_units = (DX2 ? 2 : 1) * per_phase;
  const int nch = p.Cin / 32;
  const int G = static_cast<int>(gridDim.x);
  // consecutive units on one XCD: the channel tiles of a band (and
  // neighbouring bands) read the same input rows from that XCD's L2
  const int wg = xcd_remap(static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x));
  const int my_units = wg < n_units ? (n_units - 1 - wg) / G + 1 : 0;
  const int n_stages = my_units * nch;
  // unit u: co tile fastest (the tiles of one band share its input in L2);
  // dx mode: the row phase ph slowest, so a workgroup's units cover both
  // alike
  auto unit_of = [&](int st, int &b, int &oh0, int &n0, int &ph) __attribute__((always_inline)) {
    int u = wg + (st / nch) * G;
    ph = DX2 ? u / per_phase : 0;
    if constexpr (DX2) u %= per_phase;
    n0 = (u % n_tiles) * BN;
    const int band = u / n_tiles;
    if constexpr (IPB > 1) {
      b = band * IPB;  // the band's first image (the last band may be partial)
      oh0 = 0;
    } else {
      b = band / bands_per_img;
      oh0 = (band % bands_per_img) * RB;
    }
  };

  const __amdgpu_buffer_rsrc_t x_rsrc = buffer_rsrc(p.x, p.x_bytes);
  const __amdgpu_buffer_rsrc_t w_rsrc = buffer_rsrc(p.w, p.w_bytes);
  const uint32_t smem0 = lds_address(smem);
  const int K = KH * KW * p.Cin;
  constexpr int ES = INT8B ? 1 : 2;  // bytes per weight element
  // DMA of stage st (chunk st % nch of its unit) into stage buffer st % 3:
  // instructions r NW + w; the first HINSTR fill the halo, the next WINSTR
  // the weights, and the excess ones (so that every wave issues DI) repeat
  // the first ones: the same bytes to the same place.  Each lane's source
  // offsets for the DMA cursor's unit are computed once, at its first chunk
  // (kOffNone for padding, pad slots and past the last unit); a chunk adds
  // its channel offset, which keeps kOffNone beyond every extent.
  int dma_off[DI];
  auto dma_unit = [&](int st) __attribute__((always_inline)) {
    const bool live = st < n_stages;
    int b, oh0, n0, ph;
    unit_of(st, b, oh0, n0, ph);
    // weight rows: forward [C_OUT][KH][KW][C_IN] (taps kh KW + kw); dx
    // mode, row phase a = ph: the T = a + 1 taps of phase (a, 0), then the 2 T
    // of phase (a, 1), each phase's block [C_IN][taps][C_OUT] at its offset
    const int T = ph + 1;
    const int taps = DX2 ? 3 * T : KH * KW;
#pragma unroll
    for (int r = 0; r < DI; ++r) {
      const int ins0 = r * NW + w;  // wave-uniform
      const int ins = ins0 < S::INSTR ? ins0 : ins0 - S::INSTR;
      int off = kOffNone;
      if (ins < S::HINSTR) {
        const int s = ins * 64 + lane;
        const int pix = s >> 2, pos = s & 3;
        // halo slot cs of row hr holds halo column hc (stride 2: its phase plane)
        const int hr = pix / HC, cs = pix % HC;
        const int hc = S2 ? 2 * (cs % S::PLANE) + cs / S::PLANE : cs;
        // multi-image band: halo row hr is row hr % HRI of image b + hr / HRI
        const int bi = b + (IPB > 1 ? hr / S::HRI : 0);
        const int ih = (S2 ? 2 * oh0 : oh0) - p.PH + (IPB > 1 ? hr % S::HRI : hr), iw = hc - p.PW;
        const bool ok = live & (s < S::HSLOTS) & (static_cast<unsigned>(ih) < static_cast<unsigned>(p.H)) &
                        (static_cast<unsigned>(iw) < static_cast<unsigned>(p.W)) & (bi < p.B);
        if (ok)
          off = static_cast<int>(((static_cast<int64_t>(bi) * p.H + ih) * p.W + iw) * p.Cin * 2 +
                                 16 * (pos ^ ((cs >> 2) & 3)));
      } else {
        const int s = (ins - S::HINSTR) * 64 + lane;
        const int n = s / S::RS, j = s % S::RS;
        const int tap = j / S::QT, q = j % S::QT;
        const bool ok = live & (s < S::WSLOTS) & (j < S::RS - 1) & (tap < taps);
        int64_t e = static_cast<int64_t>(n0 + n) * K + tap * p.Cin;
        if constexpr (DX2) {
          const bool c1 = tap >= T;  // phase (a, 1)
          e = p.phase_off[2 * ph + c1] + static_cast<int64_t>(n0 + n) * (c1 ? 2 * T : T) * p.Cin +
              (c1 ? tap - T : tap) * p.Cin;
        }
        if (ok) off = static_cast<int>(e * ES + 16 * q);
      }
      dma_off[r] = off;
    }
  };
  auto dma_stage = [&](int st) __attribute__((always_inline)) {
    if (st % nch == 0) dma_unit(st);
    const int c0 = (st % nch) * 32;
    const uint32_t buf = smem0 + (st % S::NSTG) * S::STAGE;
#pragma unroll
    for (int r = 0; r < DI; ++r) {
      const int ins0 = r * NW + w;  // wave-uniform
      const int ins = ins0 < S::INSTR ? ins0 : ins0 - S::INSTR;
      const bool halo = ins < S::HINSTR;
      const uint32_t dst = halo ? buf + ins * 1024 : buf + S::HBYTES + (ins - S::HINSTR) * 1024;
      buffer_lds_dma16(halo ? x_rsrc : w_rsrc, dma_off[r] + c0 * (halo ? 2 : ES), __builtin_amdgcn_readfirstlane(dst));
    }
  };

  // ── MFMA side
  // the wave's pixel block and (KS = 2) its k-step of every tap
  const int pbk = KS > 1 ? w % S::NPB : w, hk = KS > 1 ? w / S::NPB : 0;
  const int px = min(32 * pbk + c, S::NPX - 1);  // pixels past the band repeat the last one
  // halo row of the pixel's first tap (multi-image band: in its image's halo)
  constexpr int SR = S2 ? 2 : 1;
  const int pr = IPB > 1 ? (px / (RB * OWT)) * S::HRI + SR * ((px % (RB * OWT)) / OWT) : SR * (px / OWT);
  const int pc = px % OWT;
  // dx mode: one accumulator set per column phase
  constexpr int NSET = DX2 ? 2 : 1;
  f32x16 acc[NSET * NB];
#pragma unroll
  for (int i = 0; i < NSET * NB; ++i) acc[i] = zero16();
  // Weight fragment of channel block i for k-step (tap, h): bf16 straight
  // from LDS, or int8 read raw (8 bytes) and converted in registers
  typedef typename std::conditional<INT8B, u32x2, bf16x8>::type wraw_t;
  auto wread = [&](const char *wb, int i, int tap, int h) __attribute__((always_inline)) {
    const char *row = wb + (32 * i + c) * (S::RS * 16);
    if constexpr (INT8B) return *reinterpret_cast<const u32x2 *>(row + (tap * 2 + h) * 16 + 8 * g);
    else return *reinterpret_cast<const bf16x8 *>(row + (tap * 4 + 2 * h + g) * 16);
  };
  auto wconv = [&](const wraw_t &q) __attribute__((always_inline)) {
    if constexpr (INT8B) {
      bf16x8 f;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const uint32_t word = q[t >> 1] >> (16 * (t & 1));
        const bf16x2 pr2 = cvt_pk_bf16(static_cast<float>(static_cast<int8_t>(word & 0xffu)),
                                       static_cast<float>(static_cast<int8_t>((word >> 8) & 0xffu)));
        f[2 * t] = pr2[0];
        f[2 * t + 1] = pr2[1];
      }
      return f;
    } else {
      return q;
    }
  };
  // One chunk: KH*KW taps x 2 k-steps.  The fragments of k-step ks + kLA
  // are read while k-step ks multiplies (a window of kLA + 1 fragment sets):
  // with one k-step of lookahead every k-step waited for its reads behind a
  // single MFMA.  A scheduling fence per k-step keeps the compiler from
  // hoisting every read of the unrolled loop (the int8 kernel then held ~480
  // registers).
  constexpr int kLA = DX2 ? 1 : 2, kWin = kLA + 1;
  // The unit's taps: forward, tap j = (kh, kw) = (j / KW, j % KW); dx mode,
  // row phase with TT taps: j < TT is tap (j, 0) of phase (a, 0)
  // (accumulator set 0), then j - TT = 2 t + s is tap (t, s) of phase (a, 1)
  // (set 1).  Tap (t, s) reads halo pixel (pr + t, pc + s).
  auto compute_taps = [&](int st, auto tsel) __attribute__((always_inline)) {
    constexpr int TT = decltype(tsel)::value;
    constexpr int NTAP = DX2 ? 3 * TT : KH * KW;
    auto tap_set = [](int j) { return DX2 && j >= TT ? 1 : 0; };
    auto tap_dh = [](int j) { return DX2 ? (j < TT ? j : (j - TT) / 2) : j / KW; };
    auto tap_dw = [](int j) { return DX2 ? (j < TT ? 0 : (j - TT) % 2) : j % KW; };
    const char *hb = smem + (st % S::NSTG) * S::STAGE;
    const char *wb = hb + S::HBYTES;
    // the wave's k-steps i = 0 .. NKS-1: tap tap_of(i), channel half h_of(i)
    constexpr int NKS = NTAP * 2 / KS;
    auto tap_of = [](int i) { return KS > 1 ? i : i >> 1; };
    auto h_of = [&](int i) { return KS > 1 ? hk : i & 1; };
    auto xread = [&](int ks) __attribute__((always_inline)) {
      const int tap = tap_of(ks), h = h_of(ks);
      const int kh = tap_dh(tap), kw = tap_dw(tap);
      // halo column pc + kw, or (stride 2) 2 pc + kw in its phase plane
      const int cs = S2 ? (kw & 1) * S::PLANE + pc + (kw >> 1) : pc + kw;
      return *reinterpret_cast<const bf16x8 *>(hb + ((pr + kh) * HC + cs) * 64 + 16 * ((2 * h + g) ^ ((cs >> 2) & 3)));
    };
    bf16x8 xw[kWin];
    wraw_t ww[kWin][NB];
    auto fetch = [&](int ks) __attribute__((always_inline)) {
      xw[ks % kWin] = xread(ks);
#pragma unroll
      for (int i = 0; i < NB; ++i) ww[ks % kWin][i] = wread(wb, i, tap_of(ks), h_of(ks));
    };
#pragma unroll
    for (int ks = 0; ks < kLA; ++ks) fetch(ks);
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      if (ks + kLA < NKS) fetch(ks + kLA);
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        const int a = tap_set(tap_of(ks)) * NB + i;
        acc[a] = mfma32x32x16(wconv(ww[ks % kWin][i]), xw[ks % kWin], acc[a]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  auto compute_stage = [&](int st) __attribute__((always_inline)) {
    if constexpr (DX2) {
      int b, oh0, n0, ph;
      unit_of(st, b, oh0, n0, ph);
      if (ph == 0) compute_taps(st, std::integral_constant<int, 1>{});
      else compute_taps(st, std::integral_constant<int, 2>{});
    } else {
      compute_taps(st, std::integral_constant<int, 0>{});
    }
  };

  const EpiAct ea = epi_act(p.act);
  const float lo = ea.relu ? 0.0f : -INFINITY;
  // dx mode: y is dx, [B, 2 OH, 2 OWT, C]
  const __amdgpu_buffer_rsrc_t y_rsrc =
      buffer_rsrc(p.y, static_cast<int>(static_cast<int64_t>(p.B) * p.OH * OWT * p.Cout * 2 * (DX2 ? 4 : 1)));
  // dx mode: accumulator set `set` of row phase ph is phase (ph, set)
  // Epilogue of stage st's unit: 64 channels (blocks 2 hp, 2 hp + 1) at a
  // time; lane (c, g) holds channels 32 i + 8 q + 4 g + (0..3) of pixel c,
  // permlane32 swaps make 16-byte chunks 4 (i % 2) + 2 pr + g of the 128-byte
  // segment, staged at chunk position ^ (c & 7) and stored as 8 whole rows
  // per instruction.
  auto epilogue = [&](int st, auto sig, int set) __attribute__((always_inline)) {
    int b, oh0, n0, ph;
    unit_of(st, b, oh0, n0, ph);
    char *const stg = smem + (st % S::NSTG) * S::STAGE + pbk * S::STG;
    const int64_t pix0 = (static_cast<int64_t>(b) * p.OH + oh0) * OWT;  // the band's first pixel
#pragma unroll
    for (int hp = 0; hp < NB / 2; ++hp) {
#pragma unroll
      for (int ii = 0; ii < 2; ++ii) {
        const int i = 2 * hp + ii;
        // (dx mode: no scale, bias or activation)
        f32x4 em[4], ead[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if constexpr (DX2) {
            em[q] = f32x4{1.0f, 1.0f, 1.0f, 1.0f};
            ead[q] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
          } else {
            em[q] = *reinterpret_cast<const f32x4 *>(cmul + 32 * i + 8 * q + 4 * g);
            ead[q] = *reinterpret_cast<const f32x4 *>(cadd + 32 * i + 8 * q + 4 * g);
          }
        }
#pragma unroll
        for (int prr = 0; prr < 2; ++prr) {
          u32x2 hv[2];
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            const int q = 2 * prr + t;
            bf16x4 o;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              float r = __builtin_fmaf(acc[set * NB + i][4 * q + e], em[q][e], ead[q][e]);
              if constexpr (decltype(sig)::value) r = epi_sig(r, ea);
              o[e] = static_cast<bf16>(r < lo ? lo : r);
            }
            hv[t] = __builtin_bit_cast(u32x2, o);
          }
          u32x4 v;
#pragma unroll
          for (int d = 0; d < 2; ++d) {
            const auto sw = __builtin_amdgcn_permlane32_swap(hv[0][d], hv[1][d], false, false);
            v[d] = sw[0];
            v[2 + d] = sw[1];
          }
          const int k = 4 * ii + 2 * prr + g;
          *reinterpret_cast<u32x4 *>(stg + c * 128 + 16 * (k ^ (c & 7))) = v;
        }
      }
#pragma unroll
      for (int r8 = 0; r8 < 4; ++r8) {
        const int pl = 8 * r8 + (lane >> 3), k = lane & 7;
        const u32x4 v = *reinterpret_cast<const u32x4 *>(stg + pl * 128 + 16 * (k ^ (pl & 7)));
        const int pxl = 32 * pbk + pl;
        int64_t opix = pix0 + pxl;
        if constexpr (DX2) {
          // phase pixel (u, v) of phase (a, c) is dx pixel (2 u + a, 2 v + c)
          const int u = oh0 + pxl / OWT, v = pxl % OWT;
          opix = (static_cast<int64_t>(b) * 2 * p.OH + 2 * u + ph) * (2 * OWT) + 2 * v + set;
        }
        const int off = pxl < S::NPX ? static_cast<int>((opix * p.Cout + n0 + 64 * hp) * 2 + 16 * k) : kOffNone;
        __builtin_amdgcn_raw_buffer_store_b128(v, y_rsrc, off, 0, 0);
      }
    }
  };

  // coefficient table of the unit's channels (refilled when n0 changes):
  // filled by plain loads before the first DMA and at unit boundaries after
  // the stage barrier (a unit's first epilogue is nch stages later)
  auto fill_coeffs = [&](int n0) __attribute__((always_inline)) {
    for (int j = tid; j < BN; j += S::NT) {
      const int n = n0 + j;
      float m = 1.0f, a = 0.0f;
      if (p.scale != nullptr) m = p.scale[n];
      if (p.bias != nullptr) a = p.bias[n];
      if (p.bias_bf16 != nullptr) a += static_cast<float>(p.bias_bf16[n]);
      cmul[j] = m;
      cadd[j] = a;
    }
  };
  if (my_units > 0) {
    int b, oh0, n0, ph;
    unit_of(0, b, oh0, n0, ph);
    fill_coeffs(n0);
  }
  __syncthreads();

  constexpr int AHEAD = S::NSTG - 1;  // DMA passes issued ahead of the stage computed
#pragma unroll
  for (int j = 0; j < AHEAD; ++j) dma_stage(j);
  // bit k: iteration st-1-k ended a unit (issued epilogue stores)
  unsigned epi_hist = 0;
  for (int st = 0; st < n_stages; ++st) {
    // stage st landed; issued after its DMA and left in flight: the DMA of
    // the next AHEAD-1 stages and the epilogue stores of the last AHEAD
    // iterations
    const int epis = __builtin_popcount(epi_hist & ((1u << AHEAD) - 1));
    constexpr int base = (AHEAD - 1) * DI;
    if (epis == 0) __builtin_amdgcn_s_waitcnt(vm_wait(base));
    else if (epis == 1) __builtin_amdgcn_s_waitcnt(vm_wait(base + EPI_STORES));
    else __builtin_amdgcn_s_waitcnt(vm_wait(base + 2 * EPI_STORES));
    __syncthreads();
    // every wave is past stage st-1, whose buffer stage st+AHEAD reuses
    dma_stage(st + AHEAD);
    compute_stage(st);
    epi_hist <<= 1;
    if (st % nch == nch - 1) {
      __syncthreads();  // every wave has read stage st's buffer: the epilogue slices reuse it
      if constexpr (KS == 2) {
        // the second k-half's sums, after the epilogue slices, added into the first's
        f32x4 *const part = reinterpret_cast<f32x4 *>(smem + (st % S::NSTG) * S::STAGE + S::NPB * S::STG);
        if (hk == 1) {
#pragma unroll
          for (int i = 0; i < NB; ++i)
#pragma unroll
            for (int q = 0; q < 4; ++q)
              part[((pbk * NB + i) * 4 + q) * 64 + lane] =
                  f32x4{acc[i][4 * q], acc[i][4 * q + 1], acc[i][4 * q + 2], acc[i][4 * q + 3]};
        }
        __syncthreads();
        if (hk == 0) {
#pragma unroll
          for (int i = 0; i < NB; ++i)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const f32x4 v = part[((pbk * NB + i) * 4 + q) * 64 + lane];
#pragma unroll
              for (int e = 0; e < 4; ++e) acc[i][4 * q + e] += v[e];
            }
        }
      }
      if (hk == 0) {
#pragma unroll
        for (int set = 0; set < NSET; ++set) {
          if (!DX2 && ea.sig) epilogue(st, std::true_type{}, set);
          else epilogue(st, std::false_type{}, set);
        }
      }
#pragma unroll
      for (int i = 0; i < NSET * NB; ++i) acc[i] = zero16();
      // (the epilogue's stores, which the waits count: first k-half only)
      epi_hist |= hk == 0 ? 1u : 0u;
      if (st + 1 < n_stages) {
        int b2, oh2, n2, b1, oh1, n1, ph1, ph2;
        unit_of(st, b1, oh1, n1, ph1);
        unit_of(st + 1, b2, oh2, n2, ph2);
        if (n2 != n1) {
          // every wave is done with this unit's coefficients (all passed its epilogue)
          __syncthreads();
          fill_coeffs(n2);
        }
      }
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // trailing zero-source DMA
}

template <int KH, int KW, int OWT, int RB, int BN, bool INT8B, int IPB = 1, bool S2 = false>
inline bool tile_conv_fits(const GemmParams &p) {
  const int st = S2 ? 2 : 1;
  return p.KH == KH && p.KW == KW && p.SH == st && p.SW == st && p.OW == OWT && p.OH % RB == 0 &&
         (IPB == 1 || p.OH == RB) && p.PH >= 0 &&
         p.PW >= 0 && p.Cin % 32 == 0 && p.N % BN == 0 && p.ldc == p.N && p.c_ow <= 0 &&
         (reinterpret_cast<uintptr_t>(p.A) & 15) == 0 && (reinterpret_cast<uintptr_t>(p.B) & 15) == 0 &&
         (reinterpret_cast<uintptr_t>(p.C) & 15) == 0 &&
         static_cast<int64_t>(p.M) * p.N * 2 < 0x7fffffff &&
         static_cast<int64_t>(p.M / (p.OH * p.OW)) * p.H * p.W * p.Cin * 2 < 0x7fffffff &&
         static_cast<int64_t>(p.N) * p.K * (INT8B ? 1 : 2) < 0x7fffffff;
}

template <int KH, int KW, int OWT, int RB, int BN, bool INT8B, int IPB = 1, bool S2 = false, int KS = 1>
inline void launch_tile_conv(const GemmParams &p, int act, hipStream_t s) {
  using S = TileShape<KH, KW, OWT, RB, BN, INT8B, false, IPB, S2, KS>;
  auto kern = &conv_tile_kernel<KH, KW, OWT, RB, BN, INT8B, false, IPB, S2, KS>;
  static const bool attr_set = [kern] {
    return hipFuncSetAttribute(reinterpret_cast<const void *>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                               S::LDS) == hipSuccess;
  }();
  (void)attr_set;
  TileConvParams t{};
  t.x = p.A;
  t.w = p.B;
  t.scale = p.scale;
  t.bias = p.bias;
  t.bias_bf16 = p.bias_bf16;
  t.y = p.C;
  t.B = p.M / (p.OH * p.OW);
  t.H = p.H;
  t.W = p.W;
  t.Cin = p.Cin;
  t.Cout = p.N;
  t.OH = p.OH;
  t.PH = p.PH;
  t.PW = p.PW;
  t.act = act;
  t.x_bytes = static_cast<int>(static_cast<int64_t>(t.B) * p.H * p.W * p.Cin * 2);
  t.w_bytes = static_cast<int>(static_cast<int64_t>(p.N) * p.K * (INT8B ? 1 : 2));
  const int bands = IPB > 1 ? (t.B + IPB - 1) / IPB : t.B * (p.OH / RB);
  const int units = bands * (p.N / BN);
  const int grid = std::min(units, device_cu_count());
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(grid)), dim3(S::NT), S::LDS, s, t);
}

// The band-tiled kernel for this conv, if one is built for its shape: the
// 14x14, 28x28 and 7x7 bf16 3x3 convs (ResNet stages 2-4: 14x14 256 -> 256
// at batch 64 33.4 -> 22.3 us, 28x28 128 -> 128 27.9 -> 23.6 us, 7x7 512 ->
// 512 36.6 -> 31.1 us against the implicit GEMM, split four ways along K
// there).  int8 weights do not run here as int8 (the 28x28 conv: 62 us
// against 54 us for the GEMM: each converted weight fragment feeds one MFMA
// here, so the int8 -> bf16 conversion outweighs the matrix work); the int8
// conv converts its weights to a bf16 copy first and runs the bf16 kernel.
// Which band-tiled shape takes this bf16 conv: 1 (14x14), 2 (28-wide), 3
// (7x7, two images per band), 4 (stride 2 to 7x7 outputs, two images per
// band: 14x14 512 -> 512 at batch 64 35.9 -> 30.0 us against the split-K
// implicit GEMM), 5 (stride 2 to 14x14 outputs, half-image bands: 28x28
// 256 -> 256 33.5 -> 31.0 us against the implicit GEMM; 38.8 us with one
// wave per pixel block); stride 2 to 28-wide outputs (four-row bands, 28.0
// -> 49.5 us) stays on the GEMM; 0 none.
inline int tile_conv_shape(const GemmParams &p) {
  if (tile_conv_fits<3, 3, 14, 14, 64, false>(p)) return 1;
  if (tile_conv_fits<3, 3, 28, 7, 64, false>(p)) return 2;
  if (tile_conv_fits<3, 3, 7, 7, 64, false, 2>(p)) return 3;
  if (tile_conv_fits<3, 3, 7, 7, 64, false, 2, true>(p)) return 4;
  if (tile_conv_fits<3, 3, 14, 7, 64, false, 1, true>(p)) return 5;
  return 0;
}

template <bool INT8B>
inline bool try_conv_tile(const GemmParams &p, int act, hipStream_t s) {
  if constexpr (!INT8B) {
    switch (tile_conv_shape(p)) {
      case 1: launch_tile_conv<3, 3, 14, 14, 64, false>(p, act, s); return true;
      case 2: launch_tile_conv<3, 3, 28, 7, 64, false>(p, act, s); return true;
      // 7x7 images, two per band (98 pixels, four waves)
      // (with two waves per pixel block, each on half of every chunk's
      // channels: 512 -> 512 at batch 64 30.2 -> 26.1 us, stride 2 34.5 ->
      // 30.0 us, against one wave per block and SIMD)
      case 3: launch_tile_conv<3, 3, 7, 7, 64, false, 2, false, 2>(p, act, s); return true;
      case 4: launch_tile_conv<3, 3, 7, 7, 64, false, 2, true, 2>(p, act, s); return true;
      case 5: launch_tile_conv<3, 3, 14, 7, 64, false, 1, true, 2>(p, act, s); return true;
      default: break;
    }
  }
  return false;
}

// dx of a stride-2 3x3 pad-1 conv (dx = 2 OH x 2 OW) as the band-tiled
// kernel over dy with all four sub-pixel phases in one launch: units are
// (row phase a, image band, 64 input channels), each holding phases (a, 0)
// and (a, 1) in two accumulator sets (3 or 6 taps per 32 channels of dy:
// one unit per sub-pixel phase, 1 to 4 taps, took 45.8 us at 64 x 28 x 28,
// 256 -> 256), and each phase pixel (u, v) stored to dx pixel (2 u + a,
// 2 v + c).  wp holds the phases' flipped, transposed
// weights ([C_IN][taps][C_OUT] each, at phase_off, in phase order (0, 0),
// (0, 1), (1, 0), (1, 1)).
template <int OWT, int RB>
inline bool tile_dx2_fits(int B, int OH, int OW, int Kc, int N, const void *dy, const void *wp, const void *dx) {
  return OW == OWT && OH % RB == 0 && Kc % 32 == 0 && N % 64 == 0 && aligned(dy, 16) && aligned(wp, 16) &&
         aligned(dx, 16) && static_cast<int64_t>(B) * OH * OW * Kc * 2 < 0x7fffffff &&
         static_cast<int64_t>(B) * 4 * OH * OW * N * 2 < 0x7fffffff && static_cast<int64_t>(9) * N * Kc * 2 < 0x7fffffff;
}

template <int OWT, int RB>
inline void launch_tile_dx2(const bf16 *dy, const bf16 *wp, bf16 *dx, int B, int OH, int Kc, int N,
                            const int64_t *phase_off, hipStream_t s) {
  using S = TileShape<3, 3, OWT, RB, 64, false, true>;
  auto kern = &conv_tile_kernel<3, 3, OWT, RB, 64, false, true>;
  static const bool attr_set = [kern] {
    return hipFuncSetAttribute(reinterpret_cast<const void *>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                               S::LDS) == hipSuccess;
  }();
  (void)attr_set;
  TileConvParams t{};
  t.x = dy;
  t.w = wp;
  t.y = dx;
  t.B = B;
  t.H = OH;
  t.W = OWT;
  t.Cin = Kc;
  t.Cout = N;
  t.OH = OH;
  t.PH = 0;
  t.PW = 0;
  t.act = TEENY_ACT_NONE;
  t.x_bytes = static_cast<int>(static_cast<int64_t>(B) * OH * OWT * Kc * 2);
  t.w_bytes = static_cast<int>(static_cast<int64_t>(9) * N * Kc * 2);
  for (int i = 0; i < 4; ++i) t.phase_off[i] = static_cast<int>(phase_off[i]);
  const int units = 2 * B * (OH / RB) * (N / 64);
  const int grid = std::min(units, device_cu_count());
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(grid)), dim3(S::NT), S::LDS, s, t);
}

}  // namespace teeny
