// fp32 NCHW convolution by output rows, on the fp32 matrix cores, for the
// reference's own conv config (conv2d_bias_forward, kernels/teeny-kernels/
// src/nn/conv/conv2d.rs:642-764, 1 x 64 x 56 x 56, 3x3):
//
//   y[b, n, oh, ow] = act( scale[n] * sum_{ci, kh, kw} x[b, ci, oh*SH - PH + kh, ow*SW - PW + kw]
//                                      * w[n, ci, kh, kw] + bias[n] )
//
// A workgroup owns one output row (b, oh), OW <= 64 pixels as four 16-pixel
// blocks, and 16 output channels, with eight waves: wave w takes pixel block
// w % 4 and half of every chunk's input channels (w / 4), so each SIMD runs
// two waves (one would leave the barrier and LDS latencies of every chunk
// exposed); the two halves are summed through LDS at the end.  Per chunk of
// 16 input channels one LDS-DMA pass stages the KH input rows the row needs
// (each row 64 floats wide: the data at columns 4 .. 4 + W - 1, zeros around
// it, so a padding tap reads zero) and the chunk's 16 x 16 x KH x KW
// weights; four stages, the DMA three chunks ahead of the MFMAs (the
// config's 64 channels are all in flight from the start).
// v_mfma_f32_16x16x4_f32 (A 16 x 4: weights, lane l holds A[l % 16][l / 16];
// B 4 x 16: activations, lane l holds B[l / 16][l % 16]; D: lane l holds
// D[4 (l / 16) + v][l % 16]) with four accumulator chains per wave (k-steps
// round-robin, summed at the end): fp32 products and accumulation, the
// reference's sum reassociated.  LDS strides are padded so that the four
// k-lanes of a read (four input channels / four weight rows) hit distinct
// banks: channel planes of KH x 64 + 16 floats, weight rows of 16 KH KW + 4.
#pragma once

#include "common.hpp"
#include "mfma.hpp"

namespace teeny {

template <int KH, int KW>
struct F32RowShape {
  static constexpr int RW = 64;                       // floats per staged input row
  static constexpr int CPLANE = KH * RW + 16;         // floats per staged channel
  static constexpr int XSLOTS = 16 * CPLANE / 4;      // 16-byte slots of the input stage
  static constexpr int WROW = 16 * KH * KW + 4;       // floats per staged weight row
  static constexpr int WSLOTS = 16 * WROW / 4;
  static constexpr int XINSTR = (XSLOTS + 63) / 64, WINSTR = (WSLOTS + 63) / 64;
  static constexpr int INSTR = XINSTR + WINSTR;
  static constexpr int NWV = 8;                       // waves
  static constexpr int DI = (INSTR + NWV - 1) / NWV;  // DMA instructions per wave per stage
  static constexpr int XBYTES = XINSTR * 1024, WBYTES = WINSTR * 1024;
  static constexpr int STAGE = XBYTES + WBYTES;
  static constexpr int NST = 4;
  static constexpr int RED = 4 * 64 * 16;             // the second channel half's sums
  static constexpr int LDS = NST * STAGE + 1024 + RED;
  static_assert((NST - 2) * DI < 16, "vmcnt field");
};

template <int KH, int KW, int ACT>
__global__ __launch_bounds__(512) void conv_f32_row_kernel(const float *__restrict__ x, const float *__restrict__ w,
                                                           const float *__restrict__ oscale,
                                                           const float *__restrict__ bias, float *__restrict__ y,
                                                           ConvGeo q, int x_bytes, int w_bytes) {
  using S = F32RowShape<KH, KW>;
  constexpr int KHW = KH * KW;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int tid = threadIdx.x, lane = tid & 63, r = lane & 15, kk = lane >> 4;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int pb = wv & 3, half = wv >> 2;  // pixel block, channel half
  // (b, oh): consecutive rows on one XCD (the hardware deals workgroups to
  // the XCDs round-robin), so that the rows' shared halo comes from its L2
  const int row = xcd_remap(blockIdx.x, gridDim.x);
  const int oh = row % q.OH, b = row / q.OH;
  const int n0 = blockIdx.y * 16;
  const int nch = q.Cin / 16;
  const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(x, x_bytes);
  const __amdgpu_buffer_rsrc_t wr = buffer_rsrc(w, w_bytes);
  const uint32_t smem0 = lds_address(smem), dummy0 = smem0 + S::NST * S::STAGE;
  // DMA of chunk ch (input channels 16 ch ..) into stage ch % NST
  auto dma = [&](int ch) __attribute__((always_inline)) {
    const bool live = ch < nch;
    const uint32_t buf = smem0 + (ch % S::NST) * S::STAGE;
#pragma unroll
    for (int rr = 0; rr < S::DI; ++rr) {
      const int ins = rr * S::NWV + wv;
      int off = kOffNone;
      uint32_t dst = dummy0;
      if (ins < S::XINSTR) {
        const int s = ins * 64 + lane;
        const int cl = s / (S::CPLANE / 4), j = s % (S::CPLANE / 4);
        const int kh = j / (S::RW / 4), c4 = j % (S::RW / 4);  // row kh of the chunk's channel cl, 4 floats c4
        const int ih = oh * q.SH - q.PH + kh, iw = 4 * c4 - 4;
        const bool ok = live & (s < S::XSLOTS) & (kh < KH) & (static_cast<unsigned>(ih) < static_cast<unsigned>(q.H)) &
                        (iw >= 0) & (iw + 4 <= q.W);
        if (ok) off = 4 * (((b * q.Cin + 16 * ch + cl) * q.H + ih) * q.W + iw);
        dst = buf + ins * 1024;
      } else if (ins < S::INSTR) {
        const int s = (ins - S::XINSTR) * 64 + lane;
        const int n = s / (S::WROW / 4), j = s % (S::WROW / 4);
        const bool ok = live & (s < S::WSLOTS) & (j < 4 * KHW) & (n0 + n < q.Cout);
        if (ok) off = 4 * ((n0 + n) * q.Cin * KHW + 16 * ch * KHW + 4 * j);
        dst = buf + S::XBYTES + (ins - S::XINSTR) * 1024;
      }
      buffer_lds_dma16(ins < S::XINSTR ? xr : wr, off, __builtin_amdgcn_readfirstlane(dst));
    }
  };

  const int ow = 16 * pb + r;  // this lane's output pixel (B operand column)
  f32x4 acc[4];
#pragma unroll
  for (int a = 0; a < 4; ++a) acc[a] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int ch = 0; ch < S::NST - 1; ++ch) dma(ch);
  for (int ch = 0; ch < nch; ++ch) {
    // this wave's share of chunk ch landed (the next NST - 2 may fly) ...
    __builtin_amdgcn_s_waitcnt(0xF70 | ((S::NST - 2) * S::DI));
    __syncthreads();  // ... and every wave's; all are past chunk ch-1, whose stage chunk ch+NST-1 reuses
    dma(ch + S::NST - 1);
    const float *xs = reinterpret_cast<const float *>(smem + (ch % S::NST) * S::STAGE);
    const float *ws = reinterpret_cast<const float *>(smem + (ch % S::NST) * S::STAGE + S::XBYTES);
    // k-steps (tap, channel group g4 of this wave's half): A = w[n0 + r][16 ch
    // + 4 g4 + kk][tap], B = x[16 ch + 4 g4 + kk][oh + kh][ow + kw]
#pragma unroll
    for (int tap = 0; tap < KHW; ++tap) {
      const int kh = tap / KW, kw = tap % KW;
      const int col = 4 + ow * q.SW - q.PW + kw;
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        const int cl = 4 * (2 * half + g) + kk;
        const float av = ws[r * S::WROW + cl * KHW + tap];
        const float bv = xs[cl * S::CPLANE + kh * S::RW + col];
        const int a = 2 * (tap & 1) + g;
        acc[a] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc[a], 0, 0, 0);
      }
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // trailing zero-source DMA
  f32x4 sum = (acc[0] + acc[1]) + (acc[2] + acc[3]);
  // the second half's sums through LDS (a region of its own: the trailing
  // DMA may still land in the stages of other waves)
  f32x4 *red = reinterpret_cast<f32x4 *>(smem + S::NST * S::STAGE + 1024);
  if (half == 1) red[pb * 64 + lane] = sum;
  __syncthreads();
  if (half == 1) return;
  sum += red[pb * 64 + lane];
  if (ow >= q.OW) return;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int co = n0 + 4 * kk + v;
    if (co < q.Cout) {
      float val = sum[v];
      if (oscale != nullptr) val *= oscale[co];
      if (bias != nullptr) val += bias[co];
      y[b * q.ys[0] + co * q.ys[1] + oh * q.ys[2] + ow * q.ys[3]] = apply_act<ACT, false>(val);
    }
  }
}

// The row kernel takes fp32 NCHW convs with groups 1, C_IN a multiple of 16,
// a 3x3 kernel, stride 1, OW <= 64 and input rows of W <= 56 floats whose
// start is 16-byte aligned (W % 4 == 0; the staged row's columns 4 + W ..
// 63 stay zero for the right padding, W + PW <= 60), operands below 2^31
// bytes.
inline bool f32_row_fits(const ConvGeo &q, const void *x, const void *w) {
  return q.G == 1 && q.Cin % 16 == 0 && q.KH == 3 && q.KW == 3 && q.SH == 1 && q.SW == 1 && q.OW <= 64 &&
         q.W % 4 == 0 && q.W <= 56 && q.PW <= 4 && q.PH >= 0 &&
         q.xs[3] == 1 && q.xs[2] == q.W && q.ys[3] == 1 &&  // NCHW
         (reinterpret_cast<uintptr_t>(x) & 15) == 0 && (reinterpret_cast<uintptr_t>(w) & 15) == 0 &&
         static_cast<int64_t>(q.B) * q.Cin * q.H * q.W * 4 < 0x7fffffff &&
         static_cast<int64_t>(q.Cout) * q.Cin * 9 * 4 < 0x7fffffff;
}

template <int ACT>
inline void launch_f32_row_act(const float *x, const float *w, const float *oscale, const float *bias, float *y,
                               const ConvGeo &q, hipStream_t s) {
  using S = F32RowShape<3, 3>;
  auto kern = &conv_f32_row_kernel<3, 3, ACT>;
  static const bool attr_set = [kern] {
    return hipFuncSetAttribute(reinterpret_cast<const void *>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                               S::LDS) == hipSuccess;
  }();
  (void)attr_set;
  const int xb = static_cast<int>(static_cast<int64_t>(q.B) * q.Cin * q.H * q.W * 4);
  const int wb = static_cast<int>(static_cast<int64_t>(q.Cout) * q.Cin * 9 * 4);
  const dim3 grid(static_cast<unsigned>(q.B * q.OH), static_cast<unsigned>((q.Cout + 15) / 16));
  hipLaunchKernelGGL(kern, grid, dim3(64 * S::NWV), S::LDS, s, x, w, oscale, bias, y, q, xb, wb);
}

inline bool try_conv_f32_row(const float *x, const float *w, const float *bias, float *y, const ConvGeo &q, int act,
                             hipStream_t s, const float *oscale) {
  if (!f32_row_fits(q, x, w)) return false;
  switch (act) {
    case TEENY_ACT_RELU: launch_f32_row_act<TEENY_ACT_RELU>(x, w, oscale, bias, y, q, s); break;
    case TEENY_ACT_GELU_TANH: launch_f32_row_act<TEENY_ACT_GELU_TANH>(x, w, oscale, bias, y, q, s); break;
    case TEENY_ACT_SILU: launch_f32_row_act<TEENY_ACT_SILU>(x, w, oscale, bias, y, q, s); break;
    default: launch_f32_row_act<TEENY_ACT_NONE>(x, w, oscale, bias, y, q, s); break;
  }
  return true;
}

}  // namespace teeny
