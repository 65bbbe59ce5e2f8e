// Row-band convolution for stride-1 bf16 NHWC convs with 64 output channels
// whose whole weight tensor fits in LDS (the 56x56 3x3 64 -> 64 ResNet
// layers; the space-to-depth form of the 7x7/2 stem, 4x4 taps over 16
// channels, which the raw-stem mode below forms in LDS from the RGB image):
//
//   y[b, oh, ow, co] = act( scale[co] * sum_{kh, kw, ci} x[b, oh - PH + kh, ow - PW + kw, ci]
//                                        * w[co, kh, kw, ci] + bias[co] )
//
// The implicit GEMM (gemm_core.hpp) gathers a pixel's KH x KW taps from L2
// for every output tile and streams the weights once per tile: the 56x56
// 3x3 layer moves ~9x its input and ~3100 copies of its 74 KiB of weights
// through L2, and the stem ~16x its input.  Here each workgroup (one per
// CU, persistent) loads the weights into LDS once, then walks bands of RB
// whole output rows of one image: per channel chunk (CC <= 32 channels) the
// band's input rows with their halo, (RB + KH - 1) x (OW + KW - 1) pixels,
// arrive in LDS by one LDS-DMA pass (padding pixels read as zeros through
// out-of-extent buffer offsets), and every tap is then read from LDS.
//
// A band has RB * OW = 32 * NW pixels (RB = 4 at OW = 56, RB = 2 at OW =
// 112: 7 waves); wave w owns pixels 32 w .. 32 w + 31 of the band and all 64
// output channels.  v_mfma_f32_32x32x16_bf16 computes the transposed tile
// D[co][px] (weights as the A operand, 16 channels of one tap per k-step),
// so a lane's registers are 4 consecutive output channels of one pixel.
// LDS layouts: weight rows [co][(kh, kw, ci)] padded by 16 bytes (an odd
// number of 16-byte units, so the 16-byte fragment reads of 16 consecutive
// rows hit 16 disjoint bank quads); halo pixels of CC channels, the 16-byte
// chunk q of halo column hc at position q ^ ((hc >> 2) & 3) when CC = 32 (a
// fragment read touches 8 consecutive columns per quarter-wave; unswizzled,
// columns hc and hc + 4 share banks).
//
// Raw-stem mode (RAWW > 0): the DMA stages the band's raw RGB rows (2 of
// them per space-to-depth row) instead of a precomputed space-to-depth
// tensor; once a stage has landed, every thread rebuilds the s2d halo pixels
// from them (two 12-byte raw windows per pixel, shifted into place with
// alignbit), a second barrier publishes the halo, and the MFMAs read it.
// The weights' s2d form is also built at start-up from the raw 7x7 weights.
// This replaces a separate repack pass that wrote and re-read a 27 MB
// space-to-depth copy of the batch-64 input (stem 50 -> 41 us).  The s2d
// pixels hold their 12 channels with no padding (24 bytes), so a kernel
// row's 4 taps are 48 consecutive k and the MFMAs run 12 k-steps per
// output, not the 16 of 16-channel pixels (stem 38.6 -> 35.2 us).
//
// Pipeline: NHB halo buffers, the DMA NHB - 1 chunk stages ahead of the
// MFMAs, one barrier per stage (a stage's DMA is issued after the barrier
// that ends the stage which last read its buffer).  Every wave issues the
// same DMA count per stage (rounds past the halo's slots go to a 1 KiB
// dummy area), so an explicit s_waitcnt vmcnt leaves the newer stages in
// flight; the count includes the epilogue stores issued since the awaited
// DMA (vector memory operations retire in issue order), so the stores stay
// in flight too.  Epilogue: scale / bias / activation
// on the fp32 accumulators, bf16 through a per-wave 2 KiB LDS slice (32
// pixels x 32 channels at a time) and out as 16-byte chunks, 4 per pixel
// row segment.
#pragma once

#include <atomic>

#include "gemm_core.hpp"

namespace teeny {

struct BandParams {
  const bf16 *x;  // [B, H, W, CIN]; raw-stem mode: the raw image [B, H, W, 3]
  const bf16 *w;  // [64, KH, KW, CIN]; raw-stem mode: the raw 7x7 weights [64, 7, 7, 3]
  const float *scale, *bias;
  const bf16 *bias_bf16;
  bf16 *y;        // [B, OH, OW, 64]
  int B, H, W, OH, PH, PW, act;
  int x_bytes;    // byte extent of x (below 2^31)
};

template <int CIN, int KH, int KW, int OWT, int RB>
struct BandShape {
  static constexpr int COUT = 64;
  static constexpr int NPX = RB * OWT;         // pixels per band
  static constexpr int NW = NPX / 32;          // waves
  static constexpr int NT = 64 * NW;           // threads
  static constexpr int CC = CIN >= 32 ? 32 : CIN;  // channels per halo chunk
  static constexpr int NCH = CIN / CC;         // chunks per band
  static constexpr int CPP = CC / 8;           // 16-byte chunks per halo pixel
  static constexpr int HR = RB + KH - 1, HC = OWT + KW - 1;
  static constexpr int SLOTS = HR * HC * CPP;  // 16-byte halo slots per chunk
  static constexpr int INSTR = (SLOTS + 63) / 64;   // DMA instructions per chunk (workgroup)
  static constexpr int DI = (INSTR + NW - 1) / NW;  // per wave (some go to the dummy area)
  static constexpr int HBUF = INSTR * 1024;         // bytes of one halo buffer
  static constexpr int K = KH * KW * CIN;
  static constexpr int WP = K * 2 + 16;             // weight row pitch (bytes)
  static constexpr int WBYTES = COUT * WP;
  // epilogue slice per wave: both 32-channel blocks at once for the stem
  // (one LDS write-then-read round trip per band instead of two: 35.5 ->
  // 33.6 us), one at a time where the LDS is full (the 56x56 3x3 layers)
  static constexpr int STG = CIN == 16 ? 4096 : 2048;
  static_assert(NPX % 32 == 0 && NW <= 16, "a band is whole 32-pixel blocks");
  static_assert(CIN % 16 == 0 && CC % 16 == 0 && (CPP == 2 || CPP == 4), "16-channel k-steps");
  static_assert((WP / 16) % 2 == 1, "odd number of 16-byte units per weight row");
};

// Raw-stem mode (RAWW > 0, the 7x7/2 stem over RAWW-pixel RGB rows): the
// kernel reads the raw image itself and forms the space-to-depth halo in
// LDS (see conv_band_kernel).  A band's halo rows hr = 0 .. HR-1 are s2d rows
// oh0 + hr, i.e. raw rows 2 (oh0 + hr) + dy - 3, dy = 0, 1: 2 HR raw rows of
// RAWW * 6 bytes, each staged as one zero 16-byte slot, the row, and two
// zero slots (so the 12-byte window of any s2d column, read as four aligned
// dwords, stays inside zeros where it leaves the image), after one zero
// guard slot.
template <int RAWW, int HR>
struct RawShape {
  static constexpr int DATA = RAWW * 6 / 16;                // 16-byte chunks of a raw row
  static constexpr int ROW = DATA + 3;                      // slots per staged row
  static constexpr int SLOTS = 1 + 2 * HR * ROW;            // guard + rows
  static constexpr int INSTR = (SLOTS + 63) / 64;
  static constexpr int BUF = INSTR * 1024;
  static_assert(RAWW == 0 || RAWW * 6 % 16 == 0, "raw rows of whole 16-byte chunks");
};

template <int CIN, int KH, int KW, int OWT, int RB, int NHB, int RAWW = 0>
constexpr int band_lds_bytes() {
  using S = BandShape<CIN, KH, KW, OWT, RB>;
  if constexpr (RAWW > 0) {
    // raw buffers, then one s2d halo buffer
    return S::WBYTES + NHB * RawShape<RAWW, S::HR>::BUF + (S::HR * S::HC * S::CPP * 16 + 1023) / 1024 * 1024 + 1024 +
           S::NW * S::STG;
  }
  return S::WBYTES + NHB * S::HBUF + 1024 + S::NW * S::STG;
}

template <int CIN, int KH, int KW, int OWT, int RB, int NHB, int RAWW = 0>
__global__ __launch_bounds__((BandShape<CIN, KH, KW, OWT, RB>::NT), 1) void conv_band_kernel(BandParams p) {
  using S = BandShape<CIN, KH, KW, OWT, RB>;
  using R = RawShape<RAWW, S::HR>;
  constexpr bool RAW = RAWW > 0;
  constexpr int NW = S::NW, CC = S::CC, NCH = S::NCH, CPP = S::CPP, HC = S::HC;
  // DMA instructions per wave per stage: halo slots, or raw-row slots
  constexpr int DI = RAW ? (R::INSTR + NW - 1) / NW : S::DI;
  constexpr int INFLIGHT = (NHB - 2) * DI;
  static_assert(NHB >= 2 && NHB <= 4 && INFLIGHT < 16, "halo stages / vmcnt field");
  static_assert(!RAW || (CIN == 16 && KH == 4 && KW == 4 && NCH == 1), "raw mode: the 7x7/2 stem's s2d form");
  constexpr int DBUF = RAW ? R::BUF : S::HBUF;  // bytes of one DMA stage buffer
  // raw mode: s2d halo pixels of 12 channels (24 bytes, no padding), so a
  // kernel row's 4 taps are 48 consecutive k; weight rows of 4 x 48 k plus
  // one 16-byte pad (an odd number of 16-byte units)
  constexpr int kRawPix = 24, kRawWP = 4 * 48 * 2 + 16;
  static_assert(!RAW || kRawWP <= S::WP, "packed weight rows fit the weight area");
  constexpr int S2D_BYTES = RAW ? (S::HR * HC * kRawPix + 1023) / 1024 * 1024
                                : (S::HR * HC * CPP * 16 + 1023) / 1024 * 1024;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  char *const wlds = smem;
  char *const dbuf = smem + S::WBYTES;                       // DMA stage buffers
  char *const s2d = dbuf + NHB * DBUF;                       // raw mode: the one s2d halo
  char *const dummy = s2d + (RAW ? S2D_BYTES : 0);
  const int tid = threadIdx.x;
  const int lane = tid & 63, g = lane >> 5, c = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  char *const stg = dummy + 1024 + w * S::STG;

  const int bands_per_img = p.OH / RB;
  const int n_units = p.B * bands_per_img;
  const int G = static_cast<int>(gridDim.x);
  // consecutive units on one XCD: the channel tiles of a band (and
  // neighbouring bands) read the same input rows from that XCD's L2
  const int wg = xcd_remap(static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x));
  const int my_units = wg < n_units ? (n_units - 1 - wg) / G + 1 : 0;
  const int n_stages = my_units * NCH;

  // ── weights into LDS once (16-byte loads; before any DMA is in flight)
  if constexpr (RAW) {
    // the s2d form of the 7x7 weights, built here, packed: row co holds, per
    // kernel row kh2, the 4 taps kw2 x 12 channels (2 dy + dx) 3 + c, i.e.
    // k = 48 kh2 + 12 kw2 + (2 dy + dx) 3 + c holds w[co][2 kh2 + dy][2 kw2 +
    // dx][c] (zero past the 7x7 kernel)
    for (int i = tid; i < S::COUT * 16; i += S::NT) {
      const int co = i >> 4, tap = i & 15, kh2 = tap >> 2, kw2 = tap & 3;
      bf16 e[12];
#pragma unroll
      for (int ch = 0; ch < 12; ++ch) {
        const int q = ch / 3, cc = ch % 3, kh = 2 * kh2 + (q >> 1), kw = 2 * kw2 + (q & 1);
        e[ch] = (kh < 7 && kw < 7) ? p.w[((co * 7 + kh) * 7 + kw) * 3 + cc] : static_cast<bf16>(0.0f);
      }
      u32x2 v[3];
      __builtin_memcpy(v, e, 24);
      char *dst = wlds + co * kRawWP + 2 * (48 * kh2 + 12 * kw2);
#pragma unroll
      for (int j = 0; j < 3; ++j) *reinterpret_cast<u32x2 *>(dst + 8 * j) = v[j];
    }
  } else {
    constexpr int CPR = S::K / 8;  // 16-byte chunks per weight row
    for (int i = tid; i < S::COUT * CPR; i += S::NT) {
      const int co = i / CPR, j = i % CPR;
      *reinterpret_cast<u32x4 *>(wlds + co * S::WP + 16 * j) =
          *reinterpret_cast<const u32x4 *>(p.w + static_cast<int64_t>(co) * S::K + 8 * j);
    }
  }
  // epilogue coefficients of this lane's output channels: co = 32 i + 8 q + 4 g + e,
  // by unconditional buffer loads (an absent operand gets a zero extent and
  // reads zeros), so they issue as one batch with one wait
  const __amdgpu_buffer_rsrc_t s_rsrc = buffer_rsrc(p.scale, p.scale != nullptr ? 256 : 0);
  const __amdgpu_buffer_rsrc_t b_rsrc = buffer_rsrc(p.bias, p.bias != nullptr ? 256 : 0);
  const __amdgpu_buffer_rsrc_t h_rsrc = buffer_rsrc(p.bias_bf16, p.bias_bf16 != nullptr ? 128 : 0);
  const bool scaled = p.scale != nullptr;
  f32x4 mulv[2][4], addv[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int co = 32 * i + 8 * q + 4 * g + e;
        const float m = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(s_rsrc, 4 * co, 0, 0));
        const float a = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(b_rsrc, 4 * co, 0, 0));
        const uint32_t h = __builtin_amdgcn_raw_buffer_load_b16(h_rsrc, 2 * co, 0, 0);
        mulv[i][q][e] = scaled ? m : 1.0f;
        addv[i][q][e] = a + __builtin_bit_cast(float, h << 16);
      }
  // materialised here, before any DMA is issued (a later first use would
  // make the compiler's wait for these loads drain the DMA as well)
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int q = 0; q < 4; ++q) asm volatile("" : "+v"(mulv[i][q]), "+v"(addv[i][q]));
  __syncthreads();

  // ── halo DMA of stage st (unit st / NCH, chunk st % NCH) into buffer st % NHB.
  // Slot s (16 bytes) of a buffer: halo pixel s / CPP, position s % CPP,
  // holding data chunk (s % CPP) ^ swz(hc).  A wave's round r covers slots
  // [(r NW + w) 64, + 64); rounds past the halo write the dummy area.
  const __amdgpu_buffer_rsrc_t x_rsrc = buffer_rsrc(p.x, p.x_bytes);
  const uint32_t halo0 = lds_address(dbuf), dummy0 = lds_address(dummy);
  auto swz = [](int hc) { return CPP == 4 ? (hc >> 2) & 3 : 0; };
  auto dma_stage = [&](int st) __attribute__((always_inline)) {
    const bool live = st < n_stages;
    const int unit = wg + (st / NCH) * G, ch = st % NCH;
    const int b = unit / bands_per_img;
    const int oh0 = (unit % bands_per_img) * RB;
    const uint32_t buf = halo0 + (st % NHB) * DBUF;
    if constexpr (RAW) {
      // raw rows 2 oh0 - 3 + row, row = 0 .. 2 HR - 1; slot 0 and each row's
      // first and last two slots are zeros (out-of-extent offsets)
#pragma unroll
      for (int r = 0; r < DI; ++r) {
        const int base = (r * NW + w) * 64;
        const int s = base + lane - 1;
        const int row = s / R::ROW, j = s % R::ROW - 1;
        const int ih = 2 * oh0 - 3 + row;
        const bool ok = live & (s >= 0) & (base + lane < R::SLOTS) & (j >= 0) & (j < R::DATA) &
                        (static_cast<unsigned>(ih) < static_cast<unsigned>(p.H));
        const int off = ok ? static_cast<int>((static_cast<int64_t>(b) * p.H + ih) * (RAWW * 6) + 16 * j) : kOffNone;
        const uint32_t dst = base < R::SLOTS ? buf + base * 16 : dummy0;
        buffer_lds_dma16(x_rsrc, off, __builtin_amdgcn_readfirstlane(dst));
      }
      return;
    }
#pragma unroll
    for (int r = 0; r < DI; ++r) {
      const int base = (r * NW + w) * 64;  // wave-uniform
      const int s = base + lane;
      const int pix = s / CPP, pos = s % CPP;
      const int hr = pix / HC, hc = pix % HC;
      const int ih = oh0 - p.PH + hr, iw = hc - p.PW;
      const bool ok = live & (s < S::SLOTS) & (static_cast<unsigned>(ih) < static_cast<unsigned>(p.H)) &
                      (static_cast<unsigned>(iw) < static_cast<unsigned>(p.W));
      const int off = ok ? static_cast<int>(((static_cast<int64_t>(b) * p.H + ih) * p.W + iw) * CIN * 2 +
                                            (ch * CC + 8 * (pos ^ swz(hc))) * 2)
                         : kOffNone;
      const uint32_t dst = base < S::SLOTS ? buf + base * 16 : dummy0;
      buffer_lds_dma16(x_rsrc, off, __builtin_amdgcn_readfirstlane(dst));
    }
  };

  // ── MFMA side: this lane's pixel of the band and its halo position
  const int px = 32 * w + c;
  const int pr = px / OWT, pc = px % OWT;
  f32x16 acc[2] = {zero16(), zero16()};
  // raw mode: s2d halo pixel (hr, hc) from its two raw rows 2 hr + dy: the
  // 12 bytes (two pixels of three channels) of raw columns 2 hc - 3, 2 hc - 2
  // of each row, read as four aligned dwords and shifted by a half-word:
  // channels (2 dy + dx) 3 + c, 24 bytes
  auto repack = [&](int st) __attribute__((always_inline)) {
    const char *rb = dbuf + (st % NHB) * DBUF + 16;  // row 0 slot 0 (past the guard)
    for (int px = tid; px < S::HR * HC; px += S::NT) {
      const int hr = px / HC, hc = px % HC;
      uint32_t o[6];
#pragma unroll
      for (int dy = 0; dy < 2; ++dy) {
        // window start: row slot 1 (the data) + 6 (2 hc - 3) bytes = 12 hc + 16 - 18
        const uint32_t *d = reinterpret_cast<const uint32_t *>(rb + (2 * hr + dy) * (R::ROW * 16) + 12 * hc - 4);
        const uint32_t d0 = d[0], d1 = d[1], d2 = d[2], d3 = d[3];
        o[3 * dy] = __builtin_amdgcn_alignbit(d1, d0, 16);
        o[3 * dy + 1] = __builtin_amdgcn_alignbit(d2, d1, 16);
        o[3 * dy + 2] = __builtin_amdgcn_alignbit(d3, d2, 16);
      }
      char *dst = s2d + px * kRawPix;
#pragma unroll
      for (int j = 0; j < 3; ++j) *reinterpret_cast<u32x2 *>(dst + 8 * j) = u32x2{o[2 * j], o[2 * j + 1]};
    }
  };

  constexpr int kLA = 2, kWin = kLA + 1;
  auto compute_stage = [&](int st) __attribute__((always_inline)) {
    const char *hb = RAW ? s2d : dbuf + (st % NHB) * S::HBUF;
    const int ch = st % NCH;
    constexpr int HS = CC / 16;  // k-steps per tap in a chunk
    // raw mode: 3 k-steps per kernel row (48 packed k), 12 in all, against
    // the 16 of the padded 16-channel s2d form
    constexpr int NKS = RAW ? KH * 3 : KH * KW * HS;
    auto frags = [&](int ks, bf16x8 &xf, bf16x8 &w0, bf16x8 &w1) __attribute__((always_inline)) {
      if constexpr (RAW) {
        // k-step ks: kernel row kh2 = ks / 3, k 16 j .. 16 j + 15 of its 48
        // (j = ks % 3): s2d pixels pc .. pc + 3 of halo row pr + kh2 are 96
        // consecutive bytes, of which lane half g reads 16 at 32 j + 16 g
        // (8-byte aligned: two 8-byte reads)
        const int kh2 = ks / 3, j = ks % 3;
        const char *xp = hb + ((pr + kh2) * HC + pc) * kRawPix + 32 * j + 16 * g;
        const u32x2 lo = *reinterpret_cast<const u32x2 *>(xp), hi = *reinterpret_cast<const u32x2 *>(xp + 8);
        const u32x4 v = u32x4{lo[0], lo[1], hi[0], hi[1]};
        __builtin_memcpy(&xf, &v, 16);
        const int kb = 2 * (48 * kh2 + 16 * j + 8 * g);
        w0 = *reinterpret_cast<const bf16x8 *>(wlds + c * kRawWP + kb);
        w1 = *reinterpret_cast<const bf16x8 *>(wlds + (32 + c) * kRawWP + kb);
      } else {
        const int tap = ks / HS, h = ks % HS;
        const int kh = tap / KW, kw = tap % KW;
        const int hc = pc + kw;
        const int hp = (pr + kh) * HC + hc;
        xf = *reinterpret_cast<const bf16x8 *>(hb + hp * (CC * 2) + 16 * ((2 * h + g) ^ swz(hc)));
        const int kb = 2 * (tap * CIN + ch * CC + 16 * h + 8 * g);
        w0 = *reinterpret_cast<const bf16x8 *>(wlds + c * S::WP + kb);
        w1 = *reinterpret_cast<const bf16x8 *>(wlds + (32 + c) * S::WP + kb);
      }
    };
    // the fragments of k-step ks + kLA are read while k-step ks multiplies
    // (a window of kLA + 1 sets; a scheduling fence per k-step keeps that
    // order)
    bf16x8 xw[kWin], ww0[kWin], ww1[kWin];
#pragma unroll
    for (int ks = 0; ks < kLA && ks < NKS; ++ks) frags(ks, xw[ks % kWin], ww0[ks % kWin], ww1[ks % kWin]);
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      if (ks + kLA < NKS) frags(ks + kLA, xw[(ks + kLA) % kWin], ww0[(ks + kLA) % kWin], ww1[(ks + kLA) % kWin]);
      acc[0] = mfma32x32x16(ww0[ks % kWin], xw[ks % kWin], acc[0]);
      acc[1] = mfma32x32x16(ww1[ks % kWin], xw[ks % kWin], acc[1]);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  const EpiAct ea = epi_act(p.act);
  const float lo = ea.relu ? 0.0f : -INFINITY;
  const __amdgpu_buffer_rsrc_t y_rsrc =
      buffer_rsrc(p.y, static_cast<int>(static_cast<int64_t>(p.B) * p.OH * OWT * S::COUT * 2));
  // Epilogue of unit `unit`: per 32-channel block i, lane (c, g) holds
  // channels 32 i + 8 q + 4 g + (0..3) of pixel c; a v_permlane32_swap per
  // dword gives it the 16-byte chunk 2 pr + g of the pixel's 64-byte row
  // segment, staged at chunk position (2 pr + g) ^ ((c >> 1) & 3), then read
  // back as whole segments (16 lanes = 4 pixels x 64 bytes per quarter).
  auto epilogue = [&](int unit, auto sig) __attribute__((always_inline)) {
    const int b = unit / bands_per_img;
    const int oh0 = (unit % bands_per_img) * RB;
    const int64_t pix0 = (static_cast<int64_t>(b) * p.OH + oh0) * OWT + 32 * w;  // the wave's first pixel
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int prr = 0; prr < 2; ++prr) {
        u32x2 hv[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int q = 2 * prr + t;
          bf16x4 o;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float r = __builtin_fmaf(acc[i][4 * q + e], mulv[i][q][e], addv[i][q][e]);
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
        const int k = 2 * prr + g;
        *reinterpret_cast<u32x4 *>(stg + (S::STG >= 4096 ? 2048 * i : 0) + c * 64 + 16 * (k ^ ((c >> 1) & 3))) = v;
      }
      if constexpr (S::STG < 4096) {
#pragma unroll
        for (int r2 = 0; r2 < 2; ++r2) {
          const int pl = 16 * r2 + (lane >> 2), k = lane & 3;
          const u32x4 v = *reinterpret_cast<const u32x4 *>(stg + pl * 64 + 16 * (k ^ ((pl >> 1) & 3)));
          const int off = static_cast<int>(((pix0 + pl) * S::COUT + 32 * i) * 2 + 16 * k);
          __builtin_amdgcn_raw_buffer_store_b128(v, y_rsrc, off, 0, 2);
        }
      }
    }
    // 32 pixels x 64 bytes back out: round r2, lane L holds pixel 16 r2 + L / 4,
    // chunk L % 4, by non-temporal stores (cache policy nt: in the ResNet
    // step the stem 35.4 -> 33.5 us and the 56x56 3x3 24.0 -> 22.7 us)
    if constexpr (S::STG >= 4096) {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int r2 = 0; r2 < 2; ++r2) {
          const int pl = 16 * r2 + (lane >> 2), k = lane & 3;
          const u32x4 v = *reinterpret_cast<const u32x4 *>(stg + 2048 * i + pl * 64 + 16 * (k ^ ((pl >> 1) & 3)));
          const int off = static_cast<int>(((pix0 + pl) * S::COUT + 32 * i) * 2 + 16 * k);
          __builtin_amdgcn_raw_buffer_store_b128(v, y_rsrc, off, 0, 2);
        }
      }
    }
  };

  // prologue: stages 0 .. NHB-2 in flight
#pragma unroll
  for (int st = 0; st < NHB - 1; ++st) dma_stage(st);
  // The wait for stage st's DMA counts, in issue order, everything issued
  // after it: the DMAs of the NHB - 2 later stages and the epilogue stores
  // of the iterations since (EPI_STORES per epilogue; epi_hist holds which of
  // the last NHB - 1 iterations ended one).  A fixed count would make each
  // stage wait for the previous epilogue's stores to complete.
  constexpr int EPI_STORES = 4;
  static_assert(INFLIGHT + EPI_STORES * (NHB - 1) < 16, "vmcnt field");
  unsigned epi_hist = 0;
  for (int st = 0; st < n_stages; ++st) {
    // this wave's part of stage st landed (newer stages may fly), then all waves'
    switch (__builtin_popcount(epi_hist)) {
      case 0: __builtin_amdgcn_s_waitcnt(0xF70 | INFLIGHT); break;
      case 1: __builtin_amdgcn_s_waitcnt(0xF70 | (INFLIGHT + EPI_STORES)); break;
      case 2: __builtin_amdgcn_s_waitcnt(0xF70 | (INFLIGHT + 2 * EPI_STORES)); break;
      default: __builtin_amdgcn_s_waitcnt(0xF70 | (INFLIGHT + 3 * EPI_STORES)); break;
    }
    __syncthreads();
    // every wave is past stage st-1, whose buffer the DMA of st+NHB-1 reuses
    dma_stage(st + NHB - 1);
    if constexpr (RAW) {
      // every wave is past stage st-1's MFMAs too: the s2d halo is free
      repack(st);
      __syncthreads();
    }
    compute_stage(st);
    if (st % NCH == NCH - 1) {
      const int unit = wg + (st / NCH) * G;
      if (ea.sig) epilogue(unit, std::true_type{});
      else epilogue(unit, std::false_type{});
      acc[0] = zero16();
      acc[1] = zero16();
    }
    epi_hist = ((epi_hist << 1) | (st % NCH == NCH - 1 ? 1u : 0u)) & ((1u << (NHB - 1)) - 1u);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // trailing zero-source DMA
}

// Shapes the band kernel is built for: 64 output channels, stride 1, output
// width OWT with OH a multiple of RB, C_IN = CIN, all operands 16-byte
// aligned, extents below 2^31 bytes.
template <int CIN, int KH, int KW, int OWT, int RB>
inline bool band_fits(const GemmParams &p) {
  return p.N == 64 && p.Cin == CIN && p.KH == KH && p.KW == KW && p.SH == 1 && p.SW == 1 && p.OW == OWT &&
         p.OH % RB == 0 && p.PH >= 0 && p.PW >= 0 && p.ldc == 64 && p.c_ow <= 0 &&
         (reinterpret_cast<uintptr_t>(p.A) & 15) == 0 && (reinterpret_cast<uintptr_t>(p.B) & 15) == 0 &&
         (reinterpret_cast<uintptr_t>(p.C) & 15) == 0 &&
         static_cast<int64_t>(p.M) * 64 * 2 < 0x7fffffff &&
         static_cast<int64_t>(p.M / (p.OH * p.OW)) * p.H * p.W * p.Cin * 2 < 0x7fffffff;
}

template <int CIN, int KH, int KW, int OWT, int RB, int NHB>
inline void launch_band(const GemmParams &p, int act, hipStream_t s) {
  constexpr int bytes = band_lds_bytes<CIN, KH, KW, OWT, RB, NHB>();
  static_assert(bytes <= 160 * 1024, "LDS");
  auto kern = &conv_band_kernel<CIN, KH, KW, OWT, RB, NHB>;
  static const bool attr_set = [kern] {
    return hipFuncSetAttribute(reinterpret_cast<const void *>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                               bytes) == hipSuccess;
  }();
  (void)attr_set;
  BandParams b{};
  b.x = p.A;
  b.w = static_cast<const bf16 *>(p.B);
  b.scale = p.scale;
  b.bias = p.bias;
  b.bias_bf16 = p.bias_bf16;
  b.y = p.C;
  b.B = p.M / (p.OH * p.OW);
  b.H = p.H;
  b.W = p.W;
  b.OH = p.OH;
  b.PH = p.PH;
  b.PW = p.PW;
  b.act = act;
  b.x_bytes = static_cast<int>(static_cast<int64_t>(b.B) * p.H * p.W * p.Cin * 2);
  const int units = b.B * (p.OH / RB);
  const int grid = std::min(units, device_cu_count());
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(grid)), dim3(BandShape<CIN, KH, KW, OWT, RB>::NT), bytes, s,
                     b);
}

// The 7x7 stride-2 pad-3 RGB stem (3 -> 64 channels, 224-pixel rows, 112
// output columns) straight from the raw image and raw weights: the band
// kernel's raw-stem mode, no space-to-depth pass and no scratch.  x [B, H,
// 224, 3], w [64, 7, 7, 3], y [B, OH, 112, 64], OH even.
constexpr int kStemW = 224, kStemRB = 2, kStemNHB = 3;
inline bool stem_raw_fits(int B, int Cin, int Cout, int H, int W, int OH, int OW, int KH, int KW, int SH, int SW,
                          int PH, int PW, int G, const void *x, const void *w, const void *y) {
  return Cin == 3 && Cout == 64 && W == kStemW && OW == 112 && KH == 7 && KW == 7 && SH == 2 && SW == 2 && PH == 3 &&
         PW == 3 && G == 1 && OH % kStemRB == 0 && OH == (H + 2 * PH - KH) / SH + 1 && B > 0 &&
         (reinterpret_cast<uintptr_t>(x) & 15) == 0 && (reinterpret_cast<uintptr_t>(w) & 1) == 0 &&
         (reinterpret_cast<uintptr_t>(y) & 15) == 0 && static_cast<int64_t>(B) * H * W * 3 * 2 < 0x7fffffff &&
         static_cast<int64_t>(B) * OH * OW * 64 * 2 < 0x7fffffff;
}

inline void launch_stem_raw(const bf16 *x, const bf16 *w, const float *scale, const float *bias,
                            const bf16 *bias_bf16, bf16 *y, int B, int H, int OH, int act, hipStream_t s) {
  constexpr int bytes = band_lds_bytes<16, 4, 4, 112, kStemRB, kStemNHB, kStemW>();
  static_assert(bytes <= 160 * 1024, "LDS");
  auto kern = &conv_band_kernel<16, 4, 4, 112, kStemRB, kStemNHB, kStemW>;
  static const bool attr_set = [kern] {
    return hipFuncSetAttribute(reinterpret_cast<const void *>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                               bytes) == hipSuccess;
  }();
  (void)attr_set;
  BandParams b{};
  b.x = x;
  b.w = w;
  b.scale = scale;
  b.bias = bias;
  b.bias_bf16 = bias_bf16;
  b.y = y;
  b.B = B;
  b.H = H;
  b.W = kStemW;
  b.OH = OH;
  b.PH = 3;
  b.PW = 3;
  b.act = act;
  b.x_bytes = static_cast<int>(static_cast<int64_t>(B) * H * kStemW * 3 * 2);
  const int units = B * (OH / kStemRB);
  const int grid = std::min(units, device_cu_count());
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(grid)), dim3(BandShape<16, 4, 4, 112, kStemRB>::NT), bytes, s,
                     b);
}

// The band kernel for this conv (the GEMM view of a groups-1 bf16 NHWC conv),
// if one is built for its shape; returns false otherwise.
inline bool try_conv_band(const GemmParams &p, int act, hipStream_t s) {
  if (band_fits<64, 3, 3, 56, 4>(p)) {
    launch_band<64, 3, 3, 56, 4, 3>(p, act, s);
    return true;
  }
  if (band_fits<16, 4, 4, 112, 2>(p)) {
    launch_band<16, 4, 4, 112, 2, 3>(p, act, s);
    return true;
  }
  return false;
}

}  // namespace teeny
