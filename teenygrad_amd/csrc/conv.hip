// conv2d forward (+ bias, + fused activation), and the W8A16 int8-weight conv.
//
// Reference: conv2d_forward / conv2d_bias_forward,
// kernels/teeny-kernels/src/nn/conv/conv2d.rs:43-156 and :642-764 — NCHW,
// weight [C_OUT, C_IN/G, KH, KW], zero padding by masked loads (:108-127),
// accumulation over the flat (c_in_local, kh, kw) loop (:97-146), bias added
// after the loop (:740-753).
//
// Two kernel families:
//
// conv_direct: any dtype, NCHW or NHWC (strided addressing), any groups.
//   One thread per output pixel and COB output channels of one group;
//   weights are read with workgroup-uniform addresses (scalar loads,
//   broadcast), the accumulation order is the reference's (c_in_local,
//   kh, kw).  This is the fp32 NCHW path (the reference's own config) and the
//   fallback for shapes the MFMA path does not take.
//
// implicit GEMM (gemm_core.hpp): NHWC bf16 with groups == 1.  M = B*OH*OW
//   output pixels, N = C_OUT, K = KH*KW*C_IN; weights [C_OUT, KH, KW, C_IN]
//   are a plain K-contiguous [N, K] matrix and the activation tile is
//   gathered from NHWC in 16-byte chunks (C_IN % 8 == 0) or element-wise
//   (e.g. the 3-channel stem).  1x1 stride-1 unpadded convs are plain GEMMs.
//   int8 weights (W8A16) are converted to bf16 while staging into LDS and
//   the per-channel scale is applied to the fp32 accumulator.
#include <mutex>

#include "gemm_core.hpp"
#include "conv_band.hpp"
#include "conv_tile.hpp"

namespace teeny {

struct ConvGeo {
  int B, Cin, Cout, H, W, OH, OW, KH, KW, SH, SW, PH, PW, G;
  int64_t xs[4];  // strides of x in (b, c, h, w)
  int64_t ys[4];  // strides of y in (b, c, h, w)
  int64_t ws[4];  // strides of w in (co, ci_local, kh, kw)
};

template <typename WT> __device__ __forceinline__ float wload(const WT *w, int64_t i) {
  return to_f32(w[i]);
}
template <> __device__ __forceinline__ float wload<int8_t>(const int8_t *w, int64_t i) {
  return static_cast<float>(w[i]);
}

template <typename T, typename WT, int COB, int ACT>
__global__ __launch_bounds__(64) void conv_direct(const T *__restrict__ x, const WT *__restrict__ w,
                                                  const float *__restrict__ wscale,
                                                  const float *__restrict__ oscale,
                                                  const T *__restrict__ bias_t,
                                                  const float *__restrict__ bias_f,
                                                  T *__restrict__ y, ConvGeo q) {
  constexpr bool fast = !std::is_same<T, float>::value;
  const int64_t pix = static_cast<int64_t>(blockIdx.x) * 64 + threadIdx.x;
  const int64_t npix = static_cast<int64_t>(q.B) * q.OH * q.OW;
  const int co0 = blockIdx.y * COB;
  const int cin_g = q.Cin / q.G;
  const int g_idx = co0 / (q.Cout / q.G);
  const int ci0 = g_idx * cin_g;
  const bool valid = pix < npix;
  const int64_t pp = valid ? pix : 0;
  const int ow = static_cast<int>(pp % q.OW);
  const int oh = static_cast<int>((pp / q.OW) % q.OH);
  const int b = static_cast<int>(pp / (static_cast<int64_t>(q.OW) * q.OH));
  const T *xb = x + b * q.xs[0];
  float acc[COB];
#pragma unroll
  for (int j = 0; j < COB; ++j) acc[j] = 0.0f;
  for (int cl = 0; cl < cin_g; ++cl) {
    const T *xc = xb + static_cast<int64_t>(ci0 + cl) * q.xs[1];
    for (int kh = 0; kh < q.KH; ++kh) {
      const int ih = oh * q.SH + kh - q.PH;
      const bool hok = ih >= 0 && ih < q.H;
      for (int kw = 0; kw < q.KW; ++kw) {
        const int iw = ow * q.SW + kw - q.PW;
        const float xv = (valid && hok && iw >= 0 && iw < q.W)
                             ? to_f32(xc[ih * q.xs[2] + iw * q.xs[3]])
                             : 0.0f;
        const int64_t wo = cl * q.ws[1] + kh * q.ws[2] + kw * q.ws[3];
#pragma unroll
        for (int j = 0; j < COB; ++j) {
          float wv = wload(w, (co0 + j) * q.ws[0] + wo);
          if (wscale != nullptr) wv = wv * wscale[co0 + j];  // dequantize_affine: q * scale
          acc[j] = acc[j] + xv * wv;
        }
      }
    }
  }
  if (!valid) return;
#pragma unroll
  for (int j = 0; j < COB; ++j) {
    const int co = co0 + j;
    float r = acc[j];
    if (oscale != nullptr) r = r * oscale[co];  // BatchNorm scale on the accumulator
    if (bias_t != nullptr) r = r + to_f32(bias_t[co]);
    if (bias_f != nullptr) r = r + bias_f[co];
    y[b * q.ys[0] + co * q.ys[1] + oh * q.ys[2] + ow * q.ys[3]] = from_f32<T>(apply_act<ACT, fast>(r));
  }
}

template <typename T, typename WT, int ACT>
static void launch_direct_act(const T *x, const WT *w, const float *wscale, const float *oscale, const T *bias_t,
                              const float *bias_f, T *y, const ConvGeo &q, hipStream_t s) {
  const int64_t npix = static_cast<int64_t>(q.B) * q.OH * q.OW;
  const int cout_g = q.Cout / q.G;
  const dim3 blk(64);
  if (cout_g % 8 == 0) {
    hipLaunchKernelGGL((conv_direct<T, WT, 8, ACT>), dim3(cdiv(npix, 64), q.Cout / 8), blk, 0, s,
                       x, w, wscale, oscale, bias_t, bias_f, y, q);
  } else if (cout_g % 4 == 0) {
    hipLaunchKernelGGL((conv_direct<T, WT, 4, ACT>), dim3(cdiv(npix, 64), q.Cout / 4), blk, 0, s,
                       x, w, wscale, oscale, bias_t, bias_f, y, q);
  } else {
    hipLaunchKernelGGL((conv_direct<T, WT, 1, ACT>), dim3(cdiv(npix, 64), q.Cout), blk, 0, s, x,
                       w, wscale, oscale, bias_t, bias_f, y, q);
  }
}

template <typename T, typename WT>
static void launch_direct(const T *x, const WT *w, const float *wscale, const T *bias_t,
                          const float *bias_f, T *y, const ConvGeo &q, int act, hipStream_t s,
                          const float *oscale = nullptr) {
  switch (act) {
    case TEENY_ACT_RELU:
      launch_direct_act<T, WT, TEENY_ACT_RELU>(x, w, wscale, oscale, bias_t, bias_f, y, q, s);
      break;
    case TEENY_ACT_GELU_TANH:
      launch_direct_act<T, WT, TEENY_ACT_GELU_TANH>(x, w, wscale, oscale, bias_t, bias_f, y, q, s);
      break;
    case TEENY_ACT_SILU:
      launch_direct_act<T, WT, TEENY_ACT_SILU>(x, w, wscale, oscale, bias_t, bias_f, y, q, s);
      break;
    default: launch_direct_act<T, WT, TEENY_ACT_NONE>(x, w, wscale, oscale, bias_t, bias_f, y, q, s); break;
  }
}

// Validates geometry (conv2d.rs:28-42 shape rules) and fills strides for the layout.
// ── fp32 NCHW, groups == 1: implicit GEMM on the fp32 matrix cores ─────────
// y[b, n, oh, ow] = sum_k W[n, k] X[k, m] over k = (ci, tap), m = (b, oh, ow),
// with v_mfma_f32_16x16x4_f32 (D = A B, A 16 x 4, B 4 x 16; lane l holds
// A[l % 16][l / 16], B[l / 16][l % 16] and D[4 (l / 16) + v][l % 16]).  The
// weights are the A operand and the activations the B operand, so a D
// register holds 16 consecutive output pixels of one channel (coalesced
// NCHW stores).  The reference's sum over (ci, kh, kw) is reassociated
// (fp32 products and accumulation).
//
// A workgroup owns one 16 (channels) x 16 (pixels) block.  Its weight rows
// W[n0 .. n0+15][k] are contiguous in k, so they are staged in LDS by
// coalesced loads, a chunk of input channels (all taps) at a time; in the
// product, a lane reads W[n][(ci, tap)] from LDS, where four channels of
// one tap are KH*KW floats apart (row pitch = 4 mod 64 banks keeps the 64
// reads of a wave on distinct banks for odd KH*KW).  Activations are read
// straight from global memory: for one tap a lane's address advances by
// whole channel planes, and padding is resolved once per tap by an offset
// past the buffer extent (which reads zero).  The four waves split the
// channels of a chunk (wave v takes groups of four starting at 4 v, every
// 16), and their partial sums meet in LDS in a fixed order.
template <int ACT>
__global__ __launch_bounds__(256) void conv_f32_mfma(const float *__restrict__ x, const float *__restrict__ w,
                                                     const float *__restrict__ oscale,
                                                     const float *__restrict__ bias, float *__restrict__ y,
                                                     ConvGeo q, int x_bytes, int chunk, int pitch) {
  extern __shared__ __attribute__((aligned(16))) float wl[];  // [16][pitch]
  __shared__ f32x4 part[3][64];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int r = lane & 15, kk = lane >> 4;
  const int M = q.B * q.OH * q.OW;
  const int m = blockIdx.x * 16 + r;  // this lane's output pixel (B operand column)
  const int n0 = blockIdx.y * 16;
  const bool m_ok = m < M;
  const int mm = m_ok ? m : 0;
  const int ow = mm % q.OW, t = mm / q.OW, oh = t % q.OH, b = t / q.OH;
  const int ih0 = oh * q.SH - q.PH, iw0 = ow * q.SW - q.PW;
  const int HW = q.H * q.W, KHW = q.KH * q.KW;
  const int64_t K = static_cast<int64_t>(q.Cin) * KHW;
  const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(x, x_bytes);
  f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  for (int cb = 0; cb < q.Cin; cb += chunk) {
    const int ce = min(q.Cin, cb + chunk);
    const int len = (ce - cb) * KHW;  // floats per weight row in this chunk
    __syncthreads();                  // the previous chunk's LDS reads are done
    {
      // row i = tid / 16 of the block, 16 consecutive floats per step (four
      // per thread and step as one 16-byte load when the row allows it: the
      // LDS row starts at a multiple of 4 floats since pitch = 4 mod 64)
      const int i = threadIdx.x >> 4, j0 = threadIdx.x & 15;
      const int n = n0 + i;
      const int64_t src_off = static_cast<int64_t>(n < q.Cout ? n : 0) * K + static_cast<int64_t>(cb) * KHW;
      const float *src = w + src_off;
      if (((reinterpret_cast<uintptr_t>(w) >> 2) + src_off) % 4 == 0) {
        const int len4 = len & ~3;
        for (int j = 4 * j0; j < len4; j += 64) {
          f32x4 v4 = n < q.Cout ? *reinterpret_cast<const f32x4 *>(src + j) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
          *reinterpret_cast<f32x4 *>(&wl[i * pitch + j]) = v4;
        }
        for (int j = len4 + j0; j < len; j += 16) wl[i * pitch + j] = n < q.Cout ? src[j] : 0.0f;
      } else {
        for (int j = j0; j < len; j += 16) wl[i * pitch + j] = n < q.Cout ? src[j] : 0.0f;
      }
    }
    __syncthreads();
    for (int kh = 0; kh < q.KH; ++kh) {
      for (int kw = 0; kw < q.KW; ++kw) {
        const int ih = ih0 + kh, iw = iw0 + kw;
        const bool xv = m_ok & (static_cast<unsigned>(ih) < static_cast<unsigned>(q.H)) &
                        (static_cast<unsigned>(iw) < static_cast<unsigned>(q.W));
        const int tap = kh * q.KW + kw;
        // channel c0 + kk, c0 = cb + 4 wv + 16 j: activation bytes and LDS index
        int xo = 4 * ((b * q.Cin + cb + 4 * wv + kk) * HW + ih * q.W + iw);
        int li = r * pitch + (4 * wv + kk) * KHW + tap;
#pragma unroll 4
        for (int c0 = cb + 4 * wv; c0 < ce; c0 += 16) {
          const bool live = c0 + kk < ce;
          const float a = live ? wl[li] : 0.0f;
          const float bx =
              __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(xr, (live & xv) ? xo : kOffNone, 0, 0));
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a, bx, acc, 0, 0, 0);
          xo += 64 * HW;
          li += 16 * KHW;
        }
      }
    }
  }
  if (wv > 0) part[wv - 1][lane] = acc;
  __syncthreads();
  if (wv > 0 || !m_ok) return;
  acc += part[0][lane];
  acc += part[1][lane];
  acc += part[2][lane];
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int co = n0 + 4 * kk + v;
    if (co < q.Cout) {
      float val = acc[v];
      if (oscale != nullptr) val *= oscale[co];
      if (bias != nullptr) val += bias[co];
      y[b * q.ys[0] + co * q.ys[1] + oh * q.ys[2] + ow * q.ys[3]] = apply_act<ACT, false>(val);
    }
  }
}

}  // namespace teeny
#include "conv_f32_row.hpp"
namespace teeny {

// Takes an fp32 NCHW conv with groups == 1 whose input fits 32-bit byte
// offsets and whose staged weight chunk fits LDS (3x3 stride-1 convs over
// rows of <= 56 pixels: the row kernel); returns false (nothing launched)
// otherwise.
static bool try_conv_f32_mfma(const float *x, const float *w, const float *bias, float *y, const ConvGeo &q,
                              int act, hipStream_t s, const float *oscale = nullptr) {
  if (try_conv_f32_row(x, w, bias, y, q, act, s, oscale)) return true;
  const int64_t xb = static_cast<int64_t>(q.B) * q.Cin * q.H * q.W * 4;
  const int khw = q.KH * q.KW;
  if (q.G != 1 || xb >= (int64_t{1} << 31) || khw > 128) return false;
  // channels per staged chunk: a multiple of 16 (whole groups for the four
  // waves) with 16 * chunk * KH * KW floats within about 40 KiB
  int chunk = (640 / khw) / 16 * 16;
  if (chunk < 16) chunk = 16;
  if (chunk > q.Cin) chunk = q.Cin;
  int pitch = chunk * khw;
  pitch += ((4 - pitch % 64) % 64 + 64) % 64;  // pitch = 4 (mod 64)
  const size_t lds = static_cast<size_t>(16) * pitch * sizeof(float);
  static const bool attr_set = [] {
    bool ok = true;
    const void *fns[] = {reinterpret_cast<const void *>(&conv_f32_mfma<TEENY_ACT_NONE>),
                         reinterpret_cast<const void *>(&conv_f32_mfma<TEENY_ACT_RELU>),
                         reinterpret_cast<const void *>(&conv_f32_mfma<TEENY_ACT_GELU_TANH>),
                         reinterpret_cast<const void *>(&conv_f32_mfma<TEENY_ACT_SILU>)};
    for (const void *f : fns)
      ok = ok && hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, 150 * 1024) == hipSuccess;
    return ok;
  }();
  if (!attr_set || lds > 150 * 1024) return false;
  const int64_t M = static_cast<int64_t>(q.B) * q.OH * q.OW;
  const dim3 grid(static_cast<unsigned>(cdiv(M, 16)), static_cast<unsigned>(cdiv(q.Cout, 16)));
  const int xi = static_cast<int>(xb);
  switch (act) {
    case TEENY_ACT_RELU:
      hipLaunchKernelGGL(conv_f32_mfma<TEENY_ACT_RELU>, grid, dim3(256), lds, s, x, w, oscale, bias, y, q, xi, chunk,
                         pitch);
      break;
    case TEENY_ACT_GELU_TANH:
      hipLaunchKernelGGL(conv_f32_mfma<TEENY_ACT_GELU_TANH>, grid, dim3(256), lds, s, x, w, oscale, bias, y, q, xi,
                         chunk, pitch);
      break;
    case TEENY_ACT_SILU:
      hipLaunchKernelGGL(conv_f32_mfma<TEENY_ACT_SILU>, grid, dim3(256), lds, s, x, w, oscale, bias, y, q, xi, chunk,
                         pitch);
      break;
    default:
      hipLaunchKernelGGL(conv_f32_mfma<TEENY_ACT_NONE>, grid, dim3(256), lds, s, x, w, oscale, bias, y, q, xi, chunk,
                         pitch);
      break;
  }
  return true;
}

static teeny_status make_geo(int64_t B, int64_t Cin, int64_t Cout, int64_t H, int64_t W,
                             int64_t OH, int64_t OW, const teeny_conv2d_params *prm,
                             teeny_layout layout, ConvGeo *q, const char *name) {
  const std::string n(name);
  TEENY_REQUIRE(prm != nullptr, TEENY_ERR_NULL_POINTER, n + ": params");
  TEENY_REQUIRE(B >= 0 && Cin > 0 && Cout > 0 && H > 0 && W > 0 && OH >= 0 && OW >= 0,
                TEENY_ERR_SHAPE_MISMATCH, n + ": non-positive dimension");
  TEENY_REQUIRE(prm->KH > 0 && prm->KW > 0 && prm->stride_h > 0 && prm->stride_w > 0 &&
                    prm->pad_h >= 0 && prm->pad_w >= 0 && prm->groups > 0,
                TEENY_ERR_INVALID_ARGUMENT, n + ": kernel/stride/pad/groups out of range");
  TEENY_REQUIRE(Cin % prm->groups == 0 && Cout % prm->groups == 0, TEENY_ERR_SHAPE_MISMATCH,
                n + ": channels not divisible by groups");
  TEENY_REQUIRE(OH == (H + 2 * prm->pad_h - prm->KH) / prm->stride_h + 1 &&
                    OW == (W + 2 * prm->pad_w - prm->KW) / prm->stride_w + 1 &&
                    H + 2 * prm->pad_h >= prm->KH && W + 2 * prm->pad_w >= prm->KW,
                TEENY_ERR_SHAPE_MISMATCH,
                n + ": OH/OW do not match (H + 2*pad - K) / stride + 1");
  TEENY_REQUIRE(layout == TEENY_NCHW || layout == TEENY_NHWC, TEENY_ERR_INVALID_ARGUMENT,
                n + ": unknown layout");
  TEENY_REQUIRE(prm->act >= TEENY_ACT_NONE && prm->act <= TEENY_ACT_SILU,
                TEENY_ERR_INVALID_ARGUMENT, n + ": unknown activation");
  TEENY_REQUIRE(B * H * W * Cin < (1ll << 40) && B * OH * OW * Cout < (1ll << 40) &&
                    B * OH * OW <= 0x7fffffff && Cout <= 0x7fffffff,
                TEENY_ERR_SHAPE_MISMATCH, n + ": tensor too large");
  q->B = static_cast<int>(B);
  q->Cin = static_cast<int>(Cin);
  q->Cout = static_cast<int>(Cout);
  q->H = static_cast<int>(H);
  q->W = static_cast<int>(W);
  q->OH = static_cast<int>(OH);
  q->OW = static_cast<int>(OW);
  q->KH = prm->KH;
  q->KW = prm->KW;
  q->SH = prm->stride_h;
  q->SW = prm->stride_w;
  q->PH = prm->pad_h;
  q->PW = prm->pad_w;
  q->G = prm->groups;
  const int64_t cg = Cin / prm->groups;
  if (layout == TEENY_NCHW) {
    q->xs[0] = Cin * H * W; q->xs[1] = H * W; q->xs[2] = W; q->xs[3] = 1;
    q->ys[0] = Cout * OH * OW; q->ys[1] = OH * OW; q->ys[2] = OW; q->ys[3] = 1;
    q->ws[0] = cg * prm->KH * prm->KW; q->ws[1] = prm->KH * prm->KW; q->ws[2] = prm->KW; q->ws[3] = 1;
  } else {
    q->xs[0] = H * W * Cin; q->xs[1] = 1; q->xs[2] = W * Cin; q->xs[3] = Cin;
    q->ys[0] = OH * OW * Cout; q->ys[1] = 1; q->ys[2] = OW * Cout; q->ys[3] = Cout;
    q->ws[0] = prm->KH * prm->KW * cg; q->ws[1] = 1; q->ws[2] = prm->KW * cg; q->ws[3] = cg;
  }
  return TEENY_OK;
}

static GemmParams conv_gemm_params(const void *x, const void *w, const float *scale,
                                   const float *bias, const bf16 *bias_bf16, void *y,
                                   const ConvGeo &q) {
  GemmParams p{};
  p.A = static_cast<const bf16 *>(x);
  p.lda = q.Cin;
  p.B = w;
  p.ldb = static_cast<int64_t>(q.KH) * q.KW * q.Cin;
  p.C = static_cast<bf16 *>(y);
  p.ldc = q.Cout;
  p.scale = scale;
  p.bias = bias;
  p.bias_bf16 = bias_bf16;
  p.M = q.B * q.OH * q.OW;
  p.N = q.Cout;
  p.K = q.KH * q.KW * q.Cin;
  p.H = q.H; p.W = q.W; p.Cin = q.Cin; p.OH = q.OH; p.OW = q.OW;
  p.KH = q.KH; p.KW = q.KW; p.SH = q.SH; p.SW = q.SW; p.PH = q.PH; p.PW = q.PW;
  return p;
}

// ── stride-2 convs over few input channels (the 3-channel ResNet stem) ───
// A C_IN that is not a multiple of 8 forces the element-wise gather.  For
// stride 2 the conv is rewritten exactly as a stride-1 conv on the
// space-to-depth tensor
//   xs[b][u][v][(2 dy + dx) C + c] = x_pad[b][2 u + dy][2 v + dx][c]
// (4 C channels, zero-padded to C2 = a multiple of 8, so the implicit GEMM
// gathers 16-byte chunks) with a ceil(KH/2) x ceil(KW/2) kernel
//   ws[n][kh2][kw2][(2 dy + dx) C + c] = w[n][2 kh2 + dy][2 kw2 + dx][c]
// (0 where 2 kh2 + dy >= KH or 2 kw2 + dx >= KW): output (oh, ow) reads
// x_pad rows 2 (oh + kh2) + dy = 2 oh + kh, the same taps.  The two repacked
// tensors live in the caller's scratch (the stream's workspace).
// One launch for both rewrites: blocks [0, nbx) write the input, one output
// pixel per thread; the rest write the weights, one element per thread.
// Channel ch of the rewritten tensors is sub-pixel q = ch / C, channel
// c = ch % C; both are stepped along a pixel's channels instead of divided.
__global__ __launch_bounds__(256) void s2d_kernel(const bf16 *__restrict__ x, bf16 *__restrict__ xs,
                                                  const bf16 *__restrict__ w, bf16 *__restrict__ ws, int nbx,
                                                  int B, int H, int W, int C, int PH, int PW, int Hs, int Ws,
                                                  int N, int KH, int KW, int KH2, int KW2, int C2) {
  if (static_cast<int>(blockIdx.x) < nbx) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const int64_t total = static_cast<int64_t>(B) * Hs * Ws;
    if (t >= total) return;
    const int v = static_cast<int>(t % Ws);
    const int u = static_cast<int>((t / Ws) % Hs);
    const int b = static_cast<int>(t / (static_cast<int64_t>(Ws) * Hs));
    bf16 *dst = xs + t * C2;
    if (C == 3 && C2 == 16) {
      // the RGB stem: the four sub-pixels' 3 channels each, all twelve loads
      // issued before any use (clamped addresses, zeros selected for the
      // padding), then two 16-byte stores
      float val[12];
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int ih = 2 * u + (q4 >> 1) - PH, iw = 2 * v + (q4 & 1) - PW;
        const bool ok = ih >= 0 && ih < H && iw >= 0 && iw < W;
        const int64_t base = ((static_cast<int64_t>(b) * H + (ok ? ih : 0)) * W + (ok ? iw : 0)) * 3;
#pragma unroll
        for (int c3 = 0; c3 < 3; ++c3) {
          const float xv = static_cast<float>(x[base + c3]);
          val[3 * q4 + c3] = ok ? xv : 0.0f;
        }
      }
      bf16 e[16];
#pragma unroll
      for (int k = 0; k < 16; ++k) e[k] = static_cast<bf16>(k < 12 ? val[k] : 0.0f);
      u32x4 pk[2];
      __builtin_memcpy(pk, e, 32);
      reinterpret_cast<u32x4 *>(dst)[0] = pk[0];
      reinterpret_cast<u32x4 *>(dst)[1] = pk[1];
      return;
    }
    int q = 0, c = 0;  // sub-pixel and channel of output channel c0 + k
    for (int c0 = 0; c0 < C2; c0 += 8) {
      bf16 e[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        float val = 0.0f;
        if (q < 4) {
          const int ih = 2 * u + (q >> 1) - PH, iw = 2 * v + (q & 1) - PW;
          if (ih >= 0 && ih < H && iw >= 0 && iw < W)
            val = static_cast<float>(x[((static_cast<int64_t>(b) * H + ih) * W + iw) * C + c]);
          if (++c == C) {
            c = 0;
            ++q;
          }
        }
        e[k] = static_cast<bf16>(val);
      }
      u32x4 pk;
      __builtin_memcpy(&pk, e, 16);
      *reinterpret_cast<u32x4 *>(dst + c0) = pk;
    }
    return;
  }
  const int64_t t = static_cast<int64_t>(blockIdx.x - nbx) * 256 + threadIdx.x;
  const int64_t total = static_cast<int64_t>(N) * KH2 * KW2 * C2;
  if (t >= total) return;
  const int ch = static_cast<int>(t % C2);
  const int kw2 = static_cast<int>((t / C2) % KW2);
  const int kh2 = static_cast<int>((t / (static_cast<int64_t>(C2) * KW2)) % KH2);
  const int n = static_cast<int>(t / (static_cast<int64_t>(C2) * KW2 * KH2));
  float val = 0.0f;
  if (ch < 4 * C) {
    const int q = ch / C, c = ch % C;
    const int kh = 2 * kh2 + (q >> 1), kw = 2 * kw2 + (q & 1);
    if (kh < KH && kw < KW) val = static_cast<float>(w[((static_cast<int64_t>(n) * KH + kh) * KW + kw) * C + c]);
  }
  ws[t] = static_cast<bf16>(val);
}

// Scratch layout of the space-to-depth form: the rewritten input
// [B, Hs, Ws, C2], then the rewritten weights [C_OUT, KH2, KW2, C2], then the
// GEMM's own scratch, each at a 256-byte offset.
struct S2DPlan {
  ConvGeo g2;  // the stride-1 conv that the rewrite turns the call into
  size_t xs_bytes, w_off, gemm_off;
};

static size_t round256(size_t b) { return (b + 255) / 256 * 256; }

static S2DPlan s2d_plan(const ConvGeo &q) {
  S2DPlan sp;
  ConvGeo &g2 = sp.g2;
  g2 = q;
  g2.Cin = (4 * q.Cin + 7) / 8 * 8;
  g2.KH = (q.KH + 1) / 2;
  g2.KW = (q.KW + 1) / 2;
  g2.H = q.OH + g2.KH - 1;
  g2.W = q.OW + g2.KW - 1;
  g2.SH = g2.SW = 1;
  g2.PH = g2.PW = 0;
  sp.xs_bytes = static_cast<size_t>(q.B) * g2.H * g2.W * g2.Cin * sizeof(bf16);
  sp.w_off = round256(sp.xs_bytes);
  sp.gemm_off = sp.w_off + round256(static_cast<size_t>(q.Cout) * g2.KH * g2.KW * g2.Cin * sizeof(bf16));
  return sp;
}

static bool stem_raw_ok(const ConvGeo &q, const void *x, const void *w, const void *y) {
  return stem_raw_fits(q.B, q.Cin, q.Cout, q.H, q.W, q.OH, q.OW, q.KH, q.KW, q.SH, q.SW, q.PH, q.PW, q.G, x, w, y);
}

// How a groups == 1 bf16 NHWC conv maps onto the MFMA GEMM.
enum ConvPath { kConvNoMfma, kConvPlain, kConvVec, kConvS2D, kConvScalarGemm };

template <bool INT8B>
static ConvPath conv_path(const ConvGeo &q) {
  if (q.G != 1 || q.B == 0) return kConvNoMfma;
  // the vector gather addresses whole images with 32-bit byte offsets
  const bool small_image = static_cast<int64_t>(q.H) * q.W * q.Cin < (int64_t{1} << 30);
  const bool one_by_one = q.KH == 1 && q.KW == 1 && q.SH == 1 && q.SW == 1 && q.PH == 0 && q.PW == 0;
  if (INT8B) {
    // 16-byte int8 chunks: C_IN must be a multiple of 16.
    if (q.Cin % 16 != 0 || (!one_by_one && !small_image)) return kConvNoMfma;
    return one_by_one ? kConvPlain : kConvVec;
  }
  if (q.Cin % 8 == 0 && (one_by_one || small_image)) return one_by_one ? kConvPlain : kConvVec;
  if (q.Cin % 8 == 0 || q.SH != 2 || q.SW != 2) return kConvScalarGemm;
  const ConvGeo &g2 = s2d_plan(q).g2;
  return static_cast<int64_t>(g2.H) * g2.W * g2.Cin < (int64_t{1} << 30) ? kConvS2D : kConvScalarGemm;
}

// Scratch the int8 conv needs to run on the band-tiled kernel: a bf16 copy of
// its weights (0: no band-tiled shape).
static size_t tile_w8_scratch_bytes(const GemmParams &p) {
  const int64_t n = static_cast<int64_t>(p.N) * p.K;
  return tile_conv_shape(p) != 0 && n % 16 == 0 ? static_cast<size_t>(n) * 2 : 0;
}

// Scratch bytes that let a conv take its fastest plan.
template <bool INT8B>
static size_t conv_scratch_bytes(const ConvGeo &q) {
  const GemmParams p = conv_gemm_params(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, q);
  const ConvPath path = conv_path<INT8B>(q);
  switch (path) {
    case kConvPlain: return gemm_scratch_bytes<INT8B, kAPlain>(p);
    case kConvVec:
      if (INT8B && tile_w8_scratch_bytes(p) > 0) return tile_w8_scratch_bytes(p);
      // the row-band and band-tiled kernels need none
      if (!INT8B && (band_fits<64, 3, 3, 56, 4>(p) || tile_conv_shape(p) != 0)) return 0;
      return gemm_scratch_bytes<INT8B, kAConvVec>(p);
    case kConvScalarGemm: return gemm_scratch_bytes<INT8B, kAConvScalar>(p);
    case kConvS2D: {
      // (aligned operands assumed, as for every plan this reports)
      if (stem_raw_ok(q, reinterpret_cast<const void *>(16), reinterpret_cast<const void *>(16),
                      reinterpret_cast<const void *>(16)))
        return 0;
      const S2DPlan sp = s2d_plan(q);
      const GemmParams p2 = conv_gemm_params(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, sp.g2);
      return sp.gemm_off + gemm_scratch_bytes<false, kAConvVec>(p2);
    }
    default: return 0;
  }
}

// Runs the space-to-depth form of a stride-2 bf16 NHWC conv (C_IN % 8 != 0)
// in the caller's scratch.  Returns false (nothing launched) if the scratch
// is too small for the rewritten input and weights.
static bool conv_s2d_mfma(const void *x, const void *w, const float *scale, const float *bias,
                          const bf16 *bias_bf16, void *y, const ConvGeo &q, int act, hipStream_t s, Scratch scr) {
  // the RGB stem: the band kernel forms the space-to-depth input in LDS itself
  if (stem_raw_ok(q, x, w, y)) {
    launch_stem_raw(static_cast<const bf16 *>(x), static_cast<const bf16 *>(w), scale, bias, bias_bf16,
                    static_cast<bf16 *>(y), q.B, q.H, q.OH, act, s);
    return true;
  }
  const S2DPlan sp = s2d_plan(q);
  if (scr.ptr == nullptr || scr.bytes < sp.gemm_off) return false;
  const ConvGeo &g2 = sp.g2;
  bf16 *xs = static_cast<bf16 *>(scr.ptr);
  bf16 *wsd = reinterpret_cast<bf16 *>(static_cast<char *>(scr.ptr) + sp.w_off);
  const int64_t nx = static_cast<int64_t>(q.B) * g2.H * g2.W;
  const int64_t nw = static_cast<int64_t>(q.Cout) * g2.KH * g2.KW * g2.Cin;
  const int nbx = static_cast<int>((nx + 255) / 256), nbw = static_cast<int>((nw + 255) / 256);
  hipLaunchKernelGGL(s2d_kernel, dim3(static_cast<unsigned>(nbx + nbw)), dim3(256), 0, s,
                     static_cast<const bf16 *>(x), xs, static_cast<const bf16 *>(w), wsd, nbx, q.B, q.H, q.W,
                     q.Cin, q.PH, q.PW, g2.H, g2.W, q.Cout, q.KH, q.KW, g2.KH, g2.KW, g2.Cin);
  GemmParams p = conv_gemm_params(xs, wsd, scale, bias, bias_bf16, y, g2);
  if (try_conv_band(p, act, s)) return true;
  const Scratch rest{static_cast<char *>(scr.ptr) + sp.gemm_off, scr.bytes - sp.gemm_off};
  launch_gemm_mfma<false, kAConvVec>(p, act, s, rest);
  return true;
}

// Grouped bf16 NHWC conv (groups > 1) on the register-staged implicit GEMM,
// one launch for all groups: group g reads input channels [g C_IN/G, (g+1)
// C_IN/G) of each pixel (the gather's pixel stride stays C_IN), weight rows
// [g C_OUT/G, (g+1) C_OUT/G) and writes those output channels.  Taken for
// at least 16 output channels per group (fewer leave the 64-wide MFMA
// tiles mostly empty: conv_direct instead); C_IN/G % 8 == 0 gathers 16-byte
// chunks, other widths element by element.
static bool try_conv_grouped(const void *x, const void *w, const float *scale, const float *bias,
                             const bf16 *bias_bf16, void *y, const ConvGeo &q, int act, hipStream_t s) {
  const int cin_g = q.Cin / q.G, cout_g = q.Cout / q.G;
  if (q.G < 2 || q.B == 0 || cout_g < 16 || !aligned(x, 16) || !aligned(w, 16) ||
      static_cast<int64_t>(q.H) * q.W * q.Cin >= (int64_t{1} << 30))
    return false;
  GemmParams p = conv_gemm_params(x, w, scale, bias, bias_bf16, y, q);
  p.Cin = cin_g;
  p.cst = q.Cin;
  p.N = cout_g;
  p.K = q.KH * q.KW * cin_g;
  p.ldb = p.K;
  p.ldc = q.Cout;
  p.groups = q.G;
  p.g_a = cin_g;
  p.g_b = static_cast<int64_t>(cout_g) * p.K;
  p.g_c = cout_g;
  const bool one_by_one = q.KH == 1 && q.KW == 1 && q.SH == 1 && q.SW == 1 && q.PH == 0 && q.PW == 0;
  if (cin_g % 8 == 0) {
    return one_by_one ? launch_grouped_gemm<false, kAPlain>(p, act, s)
                      : launch_grouped_gemm<false, kAConvVec>(p, act, s);
  }
  return launch_grouped_gemm<false, kAConvScalar>(p, act, s);
}

// int8 -> bf16 (exact), 16 weights per thread.
__global__ __launch_bounds__(256) void w8_to_bf16(const int8_t *__restrict__ q, bf16 *__restrict__ w,
                                                  int64_t n16) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n16) return;
  const u32x4 v = reinterpret_cast<const u32x4 *>(q)[i];
  u32x4 o[2];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t word = v[j];
    const bf16x2 lo = cvt_pk_bf16(static_cast<float>(static_cast<int8_t>(word & 0xffu)),
                                  static_cast<float>(static_cast<int8_t>((word >> 8) & 0xffu)));
    const bf16x2 hi = cvt_pk_bf16(static_cast<float>(static_cast<int8_t>((word >> 16) & 0xffu)),
                                  static_cast<float>(static_cast<int8_t>(word >> 24)));
    o[j >> 1][2 * (j & 1)] = __builtin_bit_cast(uint32_t, lo);
    o[j >> 1][2 * (j & 1) + 1] = __builtin_bit_cast(uint32_t, hi);
  }
  reinterpret_cast<u32x4 *>(w)[2 * i] = o[0];
  reinterpret_cast<u32x4 *>(w)[2 * i + 1] = o[1];
}

// The int8 3x3 convs whose shape the band-tiled kernel takes: the weights
// become a bf16 copy in the scratch (int8 values are exact in bf16), and the
// bf16 kernel applies the per-channel scale in its epilogue (affine.rs:151-161
// on the accumulator, as in every W8A16 path here).  32 x 256 x 28 x 28:
// 48.0 -> 41.2 us against the int8 implicit GEMM.  False (nothing launched)
// without enough scratch.
static bool try_conv_tile_w8(GemmParams p, int act, hipStream_t s, const Scratch scr) {
  const size_t need = tile_w8_scratch_bytes(p);
  if (need == 0 || scr.ptr == nullptr || scr.bytes < need || !aligned(scr.ptr, 16)) return false;
  bf16 *wb = static_cast<bf16 *>(scr.ptr);
  const int64_t n16 = static_cast<int64_t>(need) / 32;
  hipLaunchKernelGGL(w8_to_bf16, dim3(static_cast<unsigned>(cdiv(n16, 256))), dim3(256), 0, s,
                     static_cast<const int8_t *>(p.B), wb, n16);
  p.B = wb;
  return try_conv_tile<false>(p, act, s);
}

// bf16 NHWC, groups == 1 -> MFMA implicit GEMM.  Returns false if not taken.
template <bool INT8B>
static bool try_conv_mfma(const void *x, const void *w, const float *scale, const float *bias,
                          const bf16 *bias_bf16, void *y, const ConvGeo &q, int act,
                          hipStream_t s, const Scratch scr) {
  if constexpr (!INT8B) {
    if (q.G > 1) return try_conv_grouped(x, w, scale, bias, bias_bf16, y, q, act, s);
  }
  if (!aligned(x, 16) || !aligned(w, 16)) return false;
  const ConvPath path = conv_path<INT8B>(q);
  if (path == kConvNoMfma) return false;
  if (path == kConvS2D && conv_s2d_mfma(x, w, scale, bias, bias_bf16, y, q, act, s, scr)) return true;
  GemmParams p = conv_gemm_params(x, w, scale, bias, bias_bf16, y, q);
  if constexpr (!INT8B) {
    // stride-1 convs whose weights fit in LDS: the row-band kernel
    if (path == kConvVec && try_conv_band(p, act, s)) return true;
  }
  // stride-1 3x3 convs over short rows: band tiles with streamed weights
  // (int8 weights: converted to bf16 in the scratch first)
  if constexpr (INT8B) {
    if (path == kConvVec && try_conv_tile_w8(p, act, s, scr)) return true;
  } else {
    if (path == kConvVec && try_conv_tile<false>(p, act, s)) return true;
  }
  switch (path) {
    case kConvPlain: return launch_gemm_mfma<INT8B, kAPlain>(p, act, s, scr);
    case kConvVec: return launch_gemm_mfma<INT8B, kAConvVec>(p, act, s, scr);
    default: return launch_gemm_mfma<INT8B, kAConvScalar>(p, act, s, scr);
  }
}

// `scratch_override` (non-null) replaces the stream's workspace as the
// scratch the fast plans may use.
static teeny_status conv_entry(const void *x, const void *w, const void *bias, void *y, int64_t B,
                               int64_t Cin, int64_t Cout, int64_t H, int64_t W, int64_t OH,
                               int64_t OW, const teeny_conv2d_params *prm, teeny_dtype dtype,
                               teeny_layout layout, teeny_stream stream, const char *name,
                               const Scratch *scratch_override = nullptr) {
  ConvGeo q;
  teeny_status st = make_geo(B, Cin, Cout, H, W, OH, OW, prm, layout, &q, name);
  if (st != TEENY_OK) return st;
  if (B == 0) return TEENY_OK;
  TEENY_REQUIRE(x != nullptr && w != nullptr && y != nullptr, TEENY_ERR_NULL_POINTER,
                std::string(name) + ": x/w/y");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const Scratch scr = scratch_override != nullptr ? *scratch_override : stream_scratch(s);
  if (dtype == TEENY_F32) {
    if (!(layout == TEENY_NCHW &&
          try_conv_f32_mfma(static_cast<const float *>(x), static_cast<const float *>(w),
                            static_cast<const float *>(bias), static_cast<float *>(y), q, prm->act, s))) {
      launch_direct<float, float>(static_cast<const float *>(x), static_cast<const float *>(w),
                                  nullptr, static_cast<const float *>(bias), nullptr,
                                  static_cast<float *>(y), q, prm->act, s);
    }
    return after_launch(name, s);
  }
  if (dtype == TEENY_BF16) {
    if (!(layout == TEENY_NHWC &&
          try_conv_mfma<false>(x, w, nullptr, nullptr, static_cast<const bf16 *>(bias), y, q,
                               prm->act, s, scr))) {
      launch_direct<bf16, bf16>(static_cast<const bf16 *>(x), static_cast<const bf16 *>(w),
                                nullptr, static_cast<const bf16 *>(bias), nullptr,
                                static_cast<bf16 *>(y), q, prm->act, s);
    }
    return after_launch(name, s);
  }
  return fail(TEENY_ERR_UNSUPPORTED_DTYPE, std::string(name) + ": dtype must be F32 or BF16");
}

// Conv + BatchNorm (inference, folded to a per-channel affine) + activation:
// y = act(bn_scale[c] * conv(x, w)[c] + bn_shift[c]) in the conv's own
// epilogue (fp32 accumulator, one store).  `ys` (NCHW only, may be null)
// replaces y's strides, for the reference's padded output rows.
static teeny_status conv_bn_entry(const void *x, const void *w, const float *bn_scale, const float *bn_shift,
                                  void *y, int64_t B, int64_t Cin, int64_t Cout, int64_t H, int64_t W, int64_t OH,
                                  int64_t OW, const int64_t *ys, const teeny_conv2d_params *prm, teeny_dtype dtype,
                                  teeny_layout layout, teeny_stream stream, const char *name) {
  const std::string nm(name);
  ConvGeo q;
  teeny_status st = make_geo(B, Cin, Cout, H, W, OH, OW, prm, layout, &q, name);
  if (st != TEENY_OK) return st;
  TEENY_REQUIRE(dtype == TEENY_F32 || dtype == TEENY_BF16, TEENY_ERR_UNSUPPORTED_DTYPE,
                nm + ": dtype must be F32 or BF16");
  if (ys != nullptr) {
    TEENY_REQUIRE(layout == TEENY_NCHW, TEENY_ERR_UNSUPPORTED, nm + ": output strides are for NCHW");
    // rows of one channel, channels of one image and images must not overlap
    TEENY_REQUIRE(ys[3] == 1 && ys[2] >= OW && ys[1] >= (OH - 1) * ys[2] + OW &&
                      ys[0] >= (Cout - 1) * ys[1] + (OH - 1) * ys[2] + OW,
                  TEENY_ERR_SHAPE_MISMATCH, nm + ": output strides overlap or are not row-major");
    for (int i = 0; i < 4; ++i) q.ys[i] = ys[i];
  }
  if (B == 0) return TEENY_OK;
  TEENY_REQUIRE(x != nullptr && w != nullptr && bn_scale != nullptr && bn_shift != nullptr && y != nullptr,
                TEENY_ERR_NULL_POINTER, nm + ": x/w/bn_scale/bn_shift/y");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == TEENY_F32) {
    if (!(layout == TEENY_NCHW && try_conv_f32_mfma(static_cast<const float *>(x), static_cast<const float *>(w),
                                                    bn_shift, static_cast<float *>(y), q, prm->act, s, bn_scale))) {
      launch_direct<float, float>(static_cast<const float *>(x), static_cast<const float *>(w), nullptr, nullptr,
                                  bn_shift, static_cast<float *>(y), q, prm->act, s, bn_scale);
    }
    return after_launch(name, s);
  }
  if (!(layout == TEENY_NHWC &&
        try_conv_mfma<false>(x, w, bn_scale, bn_shift, nullptr, y, q, prm->act, s, stream_scratch(s)))) {
    launch_direct<bf16, bf16>(static_cast<const bf16 *>(x), static_cast<const bf16 *>(w), nullptr, nullptr, bn_shift,
                              static_cast<bf16 *>(y), q, prm->act, s, bn_scale);
  }
  return after_launch(name, s);
}

// ── backward ────────────────────────────────────────────────────────────
// Reference: conv2d_backward_dx (conv2d.rs:171-284), conv2d_backward_dw
// (:286-397) and the combined conv2d_backward (:399-521), the RuntimeOp's
// backward kernel (:575-617).  The reference scatters with atomic adds into
// zero-initialised dx / dw; these kernels write the same sums directly (a
// gather per element), so a zero-initialised buffer ends with the same
// values and the summation order is fixed.
//
// Direct kernels (any dtype, layout, stride, padding, groups): one thread per
// dx element, taps in (co, kh, kw) order; one workgroup per dw element,
// reducing over (b, oh, ow) with a fixed tree.  bf16 NHWC dx with groups == 1
// runs on the MFMA implicit GEMM: dx is the stride-1 convolution of dy (for a
// strided conv, dy spread out with zeros to the stride) with the weights
// flipped in (kh, kw) and transposed to [C_IN, KH, KW, C_OUT], padded by
// K - 1 - pad; the flipped weights and the spread dy live in the stream
// workspace.

template <typename T>
__global__ __launch_bounds__(256) void conv_bwd_dx_direct(const T *__restrict__ dy, const T *__restrict__ w,
                                                          T *__restrict__ dx, ConvGeo q, int nhwc) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t total = static_cast<int64_t>(q.B) * q.Cin * q.H * q.W;
  if (e >= total) return;
  int b, ci, ih, iw;
  if (nhwc) {
    ci = static_cast<int>(e % q.Cin);
    iw = static_cast<int>((e / q.Cin) % q.W);
    ih = static_cast<int>((e / (static_cast<int64_t>(q.Cin) * q.W)) % q.H);
    b = static_cast<int>(e / (static_cast<int64_t>(q.Cin) * q.W * q.H));
  } else {
    iw = static_cast<int>(e % q.W);
    ih = static_cast<int>((e / q.W) % q.H);
    ci = static_cast<int>((e / (static_cast<int64_t>(q.W) * q.H)) % q.Cin);
    b = static_cast<int>(e / (static_cast<int64_t>(q.W) * q.H * q.Cin));
  }
  const int cin_g = q.Cin / q.G, cout_g = q.Cout / q.G;
  const int g = ci / cin_g, cl = ci % cin_g;
  float acc = 0.0f;
  for (int co = g * cout_g; co < (g + 1) * cout_g; ++co) {
    for (int kh = 0; kh < q.KH; ++kh) {
      const int th = ih + q.PH - kh;
      if (th < 0 || th % q.SH != 0 || th / q.SH >= q.OH) continue;
      const int oh = th / q.SH;
      for (int kw = 0; kw < q.KW; ++kw) {
        const int tw = iw + q.PW - kw;
        if (tw < 0 || tw % q.SW != 0 || tw / q.SW >= q.OW) continue;
        const int ow = tw / q.SW;
        acc += to_f32(dy[b * q.ys[0] + co * q.ys[1] + oh * q.ys[2] + ow * q.ys[3]]) *
               to_f32(w[co * q.ws[0] + cl * q.ws[1] + kh * q.ws[2] + kw * q.ws[3]]);
      }
    }
  }
  dx[b * q.xs[0] + ci * q.xs[1] + ih * q.xs[2] + iw * q.xs[3]] = from_f32<T>(acc);
}

// dw[co, cl, kh, kw] = sum over (b, oh, ow) of dy[b, co, oh, ow] * x[b, ci, ih, iw]:
// one workgroup per weight element, a strided per-thread sum, then a fixed tree.
template <typename T>
__global__ __launch_bounds__(256) void conv_bwd_dw_direct(const T *__restrict__ dy, const T *__restrict__ x,
                                                          T *__restrict__ dw, ConvGeo q) {
  __shared__ float red[4];
  const int cin_g = q.Cin / q.G, cout_g = q.Cout / q.G;
  const int64_t id = blockIdx.x;
  const int kw = static_cast<int>(id % q.KW), kh = static_cast<int>((id / q.KW) % q.KH);
  const int cl = static_cast<int>((id / (static_cast<int64_t>(q.KW) * q.KH)) % cin_g);
  const int co = static_cast<int>(id / (static_cast<int64_t>(q.KW) * q.KH * cin_g));
  const int ci = (co / cout_g) * cin_g + cl;
  const int64_t npix = static_cast<int64_t>(q.B) * q.OH * q.OW;
  float acc = 0.0f;
  for (int64_t p = threadIdx.x; p < npix; p += 256) {
    const int ow = static_cast<int>(p % q.OW), oh = static_cast<int>((p / q.OW) % q.OH);
    const int b = static_cast<int>(p / (static_cast<int64_t>(q.OW) * q.OH));
    const int ih = oh * q.SH - q.PH + kh, iw = ow * q.SW - q.PW + kw;
    if (ih < 0 || ih >= q.H || iw < 0 || iw >= q.W) continue;
    acc += to_f32(dy[b * q.ys[0] + co * q.ys[1] + oh * q.ys[2] + ow * q.ys[3]]) *
           to_f32(x[b * q.xs[0] + ci * q.xs[1] + ih * q.xs[2] + iw * q.xs[3]]);
  }
  acc = wave_sum(acc);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0)
    dw[co * q.ws[0] + cl * q.ws[1] + kh * q.ws[2] + kw * q.ws[3]] = from_f32<T>(((red[0] + red[1]) + red[2]) + red[3]);
}

// w [C_OUT, KH, KW, C_IN] -> wt [C_IN, KH, KW, C_OUT], flipped in (kh, kw).
__global__ __launch_bounds__(256) void conv_bwd_flip_weights(const bf16 *__restrict__ w, bf16 *__restrict__ wt,
                                                             int Cout, int KH, int KW, int Cin) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t total = static_cast<int64_t>(Cout) * KH * KW * Cin;
  if (t >= total) return;
  const int co = static_cast<int>(t % Cout);
  const int kw = static_cast<int>((t / Cout) % KW);
  const int kh = static_cast<int>((t / (static_cast<int64_t>(Cout) * KW)) % KH);
  const int ci = static_cast<int>(t / (static_cast<int64_t>(Cout) * KW * KH));
  wt[t] = w[((static_cast<int64_t>(co) * KH + (KH - 1 - kh)) * KW + (KW - 1 - kw)) * Cin + ci];
}

// Weight re-layouts for dx, as a per-tap transpose: for source tap kk = kh KW
// + kw, dst[D[kk] + ci R[kk] + co] = w[co][kk][ci].  A workgroup moves one
// 64 x 64 (co, ci) tile of one tap through LDS: 16-byte reads along ci and
// 16-byte writes along co (one element per thread, as in the kernels above
// and below, reads one 2-byte value per cache line: 6-7 us for the 1.2 MB of
// a 3x3 256 -> 256 conv).  C_IN and C_OUT are multiples of 8, the pointers
// 16-byte aligned.
constexpr int kMaxTransposeTaps = 64;
struct TapMap {
  int64_t D[kMaxTransposeTaps];
  int R[kMaxTransposeTaps];
};
__global__ __launch_bounds__(256) void conv_weight_tap_transpose(const bf16 *__restrict__ w, bf16 *__restrict__ dst,
                                                                 int Cout, int KHW, int Cin, TapMap m) {
  __shared__ bf16 tile[64][64 + 8];  // [ci][co]
  const int kk = blockIdx.z;
  const int co0 = blockIdx.x * 64, ci0 = blockIdx.y * 64;
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int idx = threadIdx.x + 256 * r;
    const int co = idx >> 3, ch = idx & 7;
    const int gco = co0 + co, gci = ci0 + 8 * ch;
    u32x4 v = u32x4{0u, 0u, 0u, 0u};
    if (gco < Cout && gci < Cin)
      v = *reinterpret_cast<const u32x4 *>(w + (static_cast<int64_t>(gco) * KHW + kk) * Cin + gci);
    bf16 e[8];
    __builtin_memcpy(e, &v, 16);
#pragma unroll
    for (int j = 0; j < 8; ++j) tile[8 * ch + j][co] = e[j];
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int idx = threadIdx.x + 256 * r;
    const int ci = idx >> 3, ch = idx & 7;
    const int gci = ci0 + ci, gco = co0 + 8 * ch;
    if (gci < Cin && gco < Cout)
      *reinterpret_cast<u32x4 *>(dst + m.D[kk] + static_cast<int64_t>(gci) * m.R[kk] + gco) =
          *reinterpret_cast<const u32x4 *>(&tile[ci][8 * ch]);
  }
}
static bool tap_transpose_ok(const ConvGeo &q, const void *w, const void *dst) {
  return q.KH * q.KW <= kMaxTransposeTaps && q.Cin % 8 == 0 && q.Cout % 8 == 0 && aligned(w, 16) &&
         aligned(dst, 16);
}
static void launch_tap_transpose(const bf16 *w, bf16 *dst, const ConvGeo &q, const TapMap &m, hipStream_t s) {
  hipLaunchKernelGGL(conv_weight_tap_transpose,
                     dim3(static_cast<unsigned>(cdiv(q.Cout, 64)), static_cast<unsigned>(cdiv(q.Cin, 64)),
                          static_cast<unsigned>(q.KH * q.KW)),
                     dim3(256), 0, s, w, dst, q.Cout, q.KH * q.KW, q.Cin, m);
}

// dy [B, OH, OW, C] spread to [B, HD, WD, C] with zeros between (stride SH, SW).
__global__ __launch_bounds__(256) void conv_bwd_spread(const bf16 *__restrict__ dy, bf16 *__restrict__ dyd, int B,
                                                       int OH, int OW, int C, int HD, int WD, int SH, int SW) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;  // one 16-byte chunk (8 channels)
  const int cv = C / 8;
  const int64_t total = static_cast<int64_t>(B) * HD * WD * cv;
  if (t >= total) return;
  const int c8 = static_cast<int>(t % cv);
  const int wd = static_cast<int>((t / cv) % WD);
  const int hd = static_cast<int>((t / (static_cast<int64_t>(cv) * WD)) % HD);
  const int b = static_cast<int>(t / (static_cast<int64_t>(cv) * WD * HD));
  u32x4 v = {0u, 0u, 0u, 0u};
  if (hd % SH == 0 && wd % SW == 0 && hd / SH < OH && wd / SW < OW)
    v = *reinterpret_cast<const u32x4 *>(dy + ((static_cast<int64_t>(b) * OH + hd / SH) * OW + wd / SW) * C + 8 * c8);
  reinterpret_cast<u32x4 *>(dyd)[t] = v;
}

// ── strided dx as sub-pixel phases ──
// For stride S along an axis, the dx rows i = S u + a (phase a = 0 .. S-1)
// receive only the taps k = k0 + S t with k0 = (a + P) mod S:
//   dx[S u + a] = sum_t dy[u + d - t] w[k0 + S t],   d = (a + P - k0) / S,
// a stride-1 convolution of dy with the T = ceil((K - k0) / S) taps of that
// residue, flipped (t' = T - 1 - t reads dy row u - (T - 1 - d) + t').  Each
// of the SH x SW phases is one implicit GEMM over dy (M = B U V pixels of the
// phase, N = C_IN, K = T_h T_w C_OUT) whose output rows are every SH-th row
// and SW-th column of dx (GemmParams::c_ow remap).  Exactly the KH x KW taps
// per dx pixel: the zero-spread form executes SH SW times as many MACs.
// A phase with no taps (T = 0, e.g. odd rows of a 1x1 stride-2 conv) is zero.
struct DxAxis {
  int k0, T, pad, U;  // first tap, taps, stride-1 padding, phase extent
};
static DxAxis dx_axis(int a, int S, int P, int K, int In) {
  DxAxis x;
  x.k0 = (a + P) % S;
  x.T = x.k0 < K ? (K - x.k0 + S - 1) / S : 0;
  const int d = (a + P - x.k0) / S;
  x.pad = x.T - 1 - d;
  x.U = a < In ? (In - a + S - 1) / S : 0;
  return x;
}
constexpr int kMaxDxPhases = 16;  // SH, SW <= 4
struct DxPhaseTable {
  int SH, SW;
  int T[4], k0h[4], S[4], k0w[4];  // per row phase a: taps T, first k0h; per column phase c
  int64_t off[kMaxDxPhases];         // element offset of phase (a, c)'s weights
};
// w [C_OUT, KH, KW, C_IN] -> per phase (a, c): wp[ci][t'][s'][co] =
// w[co][k0h + SH (T - 1 - t')][k0w + SW (S - 1 - s')][ci], one thread per
// element of wp (consecutive threads write consecutive co: coalesced; the
// gathered reads hit L2).  Every weight belongs to exactly one phase, so wp
// has as many elements as w.
__global__ __launch_bounds__(256) void conv_dx_phase_weights(const bf16 *__restrict__ w, bf16 *__restrict__ wp,
                                                             int Cout, int KH, int KW, int Cin, DxPhaseTable tb) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t total = static_cast<int64_t>(Cout) * KH * KW * Cin;
  if (t >= total) return;
  // the phase (a, c) whose block [off, off + Cin T S Cout) holds t
  int a = 0, c = 0;
  for (int i = 0; i < tb.SH; ++i)
    for (int j = 0; j < tb.SW; ++j) {
      const int64_t n = static_cast<int64_t>(Cin) * tb.T[i] * tb.S[j] * Cout;
      if (n > 0 && t >= tb.off[i * tb.SW + j] && t < tb.off[i * tb.SW + j] + n) {
        a = i;
        c = j;
      }
    }
  const int T = tb.T[a], S = tb.S[c];
  int64_t r = t - tb.off[a * tb.SW + c];
  const int co = static_cast<int>(r % Cout);
  r /= Cout;
  const int sp = static_cast<int>(r % S);
  r /= S;
  const int tp = static_cast<int>(r % T);
  const int ci = static_cast<int>(r / T);
  const int kh = tb.k0h[a] + tb.SH * (T - 1 - tp), kw = tb.k0w[c] + tb.SW * (S - 1 - sp);
  wp[t] = w[((static_cast<int64_t>(co) * KH + kh) * KW + kw) * Cin + ci];
}
// Zeroes the dx pixels of the phases with no taps (mask bit a * SW + c), one
// 16-byte chunk (8 channels) per thread.
__global__ __launch_bounds__(256) void conv_dx_zero_phases(bf16 *__restrict__ dx, int B, int H, int W, int C, int SH,
                                                           int SW, unsigned mask) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int cv = C / 8;
  const int64_t total = static_cast<int64_t>(B) * H * W * cv;
  if (t >= total) return;
  const int iw = static_cast<int>((t / cv) % W);
  const int ih = static_cast<int>((t / (static_cast<int64_t>(cv) * W)) % H);
  if ((mask >> ((ih % SH) * SW + iw % SW)) & 1u) reinterpret_cast<u32x4 *>(dx)[t] = u32x4{0u, 0u, 0u, 0u};
}

struct DxPhasePlan {
  bool ok = false;
  DxAxis ah[4], aw[4];
  DxPhaseTable tb{};
  unsigned zero_mask = 0;
  size_t w_bytes = 0, gemm_off = 0;
};
static DxPhasePlan dx_phase_plan(const ConvGeo &q) {
  DxPhasePlan d;
  if (q.G != 1 || q.SH > 4 || q.SW > 4 || (q.SH == 1 && q.SW == 1) || q.Cout % 8 != 0 || q.Cin % 8 != 0 ||
      static_cast<int64_t>(q.OH) * q.OW * q.Cout >= (int64_t{1} << 30))
    return d;
  d.tb.SH = q.SH;
  d.tb.SW = q.SW;
  int64_t off = 0;
  for (int a = 0; a < q.SH; ++a) {
    d.ah[a] = dx_axis(a, q.SH, q.PH, q.KH, q.H);
    d.tb.T[a] = d.ah[a].T;
    d.tb.k0h[a] = d.ah[a].k0;
  }
  for (int c = 0; c < q.SW; ++c) {
    d.aw[c] = dx_axis(c, q.SW, q.PW, q.KW, q.W);
    d.tb.S[c] = d.aw[c].T;
    d.tb.k0w[c] = d.aw[c].k0;
  }
  for (int a = 0; a < q.SH; ++a)
    for (int c = 0; c < q.SW; ++c) {
      d.tb.off[a * q.SW + c] = off;
      const int64_t taps = static_cast<int64_t>(d.ah[a].T) * d.aw[c].T;
      off += taps * q.Cin * q.Cout;
      if (taps == 0 && d.ah[a].U > 0 && d.aw[c].U > 0) d.zero_mask |= 1u << (a * q.SW + c);
    }
  d.w_bytes = static_cast<size_t>(off) * sizeof(bf16);
  d.gemm_off = round256(d.w_bytes);
  d.ok = true;
  return d;
}
// The implicit GEMM of phase (a, c): A = dy as an NHWC image [OH, OW, C_OUT],
// B = the phase's weights, C = dx rows (S_H u + a, S_W v + c).
static GemmParams dx_phase_gemm(const DxPhasePlan &d, int a, int c, const void *dy, const bf16 *wp, void *dx,
                                const ConvGeo &q) {
  const DxAxis &h = d.ah[a], &w = d.aw[c];
  GemmParams p{};
  p.A = static_cast<const bf16 *>(dy);
  p.lda = q.Cout;
  p.B = wp + d.tb.off[a * q.SW + c];
  p.ldb = static_cast<int64_t>(h.T) * w.T * q.Cout;
  p.C = static_cast<bf16 *>(dx) + (static_cast<int64_t>(a) * q.W + c) * q.Cin;
  p.M = q.B * h.U * w.U;
  p.N = q.Cin;
  p.K = h.T * w.T * q.Cout;
  p.H = q.OH; p.W = q.OW; p.Cin = q.Cout; p.OH = h.U; p.OW = w.U;
  p.KH = h.T; p.KW = w.T; p.SH = 1; p.SW = 1; p.PH = h.pad; p.PW = w.pad;
  p.c_ow = w.U;
  p.c_oh = h.U;
  p.c_sb = static_cast<int64_t>(q.H) * q.W * q.Cin;
  p.c_su = static_cast<int64_t>(q.SH) * q.W * q.Cin;
  p.c_sv = static_cast<int64_t>(q.SW) * q.Cin;
  return p;
}
static size_t dx_phase_scratch_bytes(const ConvGeo &q) {
  const DxPhasePlan d = dx_phase_plan(q);
  if (!d.ok) return 0;
  size_t g = 0;
  for (int a = 0; a < q.SH; ++a)
    for (int c = 0; c < q.SW; ++c)
      if (d.ah[a].T > 0 && d.aw[c].T > 0 && d.ah[a].U > 0 && d.aw[c].U > 0)
        g = std::max(g, gemm_scratch_bytes<false, kAConvVec>(dx_phase_gemm(d, a, c, nullptr, nullptr, nullptr, q)));
  return d.gemm_off + g;
}
// bf16 NHWC dx of a strided conv as its sub-pixel phases; false (nothing
// launched) if it does not apply.
static bool conv_dx_phases(const void *dy, const void *w, void *dx, const ConvGeo &q, hipStream_t s, Scratch scr) {
  const DxPhasePlan d = dx_phase_plan(q);
  if (!d.ok || scr.ptr == nullptr || scr.bytes < d.gemm_off || !aligned(dy, 16) || !aligned(w, 16) ||
      !aligned(dx, 16) || !aligned(scr.ptr, 16))
    return false;
  bf16 *wp = static_cast<bf16 *>(scr.ptr);
  const int64_t nw = static_cast<int64_t>(q.Cout) * q.KH * q.KW * q.Cin;
  if (tap_transpose_ok(q, w, wp)) {
    // source tap (kh, kw) is tap (t', s') of phase (a, c), a = (kh - P_H) mod S_H
    TapMap m{};
    for (int kh = 0; kh < q.KH; ++kh)
      for (int kw = 0; kw < q.KW; ++kw) {
        const int a = ((kh - q.PH) % q.SH + q.SH) % q.SH, c = ((kw - q.PW) % q.SW + q.SW) % q.SW;
        const int T = d.tb.T[a], S = d.tb.S[c];
        const int tp = T - 1 - (kh - d.tb.k0h[a]) / q.SH, sp = S - 1 - (kw - d.tb.k0w[c]) / q.SW;
        m.D[kh * q.KW + kw] = d.tb.off[a * q.SW + c] + static_cast<int64_t>(tp * S + sp) * q.Cout;
        m.R[kh * q.KW + kw] = T * S * q.Cout;
      }
    launch_tap_transpose(static_cast<const bf16 *>(w), wp, q, m, s);
  } else {
    hipLaunchKernelGGL(conv_dx_phase_weights, dim3(static_cast<unsigned>(cdiv(nw, 256))), dim3(256), 0, s,
                       static_cast<const bf16 *>(w), wp, q.Cout, q.KH, q.KW, q.Cin, d.tb);
  }
  if (d.zero_mask != 0) {
    const int64_t nc = static_cast<int64_t>(q.B) * q.H * q.W * (q.Cin / 8);
    hipLaunchKernelGGL(conv_dx_zero_phases, dim3(static_cast<unsigned>(cdiv(nc, 256))), dim3(256), 0, s,
                       static_cast<bf16 *>(dx), q.B, q.H, q.W, q.Cin, q.SH, q.SW, d.zero_mask);
  }
  // the stride-2 3x3 pad-1 convs with 14- or 28-wide dy: all four phases
  // (1, 2, 2 and 4 taps, none padded) in one band-tiled launch
  const bool s2k3 = q.KH == 3 && q.KW == 3 && q.SH == 2 && q.SW == 2 && q.PH == 1 && q.PW == 1 &&
                    q.H == 2 * q.OH && q.W == 2 * q.OW;
  if (s2k3 && d.zero_mask == 0) {
    const bf16 *dyb = static_cast<const bf16 *>(dy);
    bf16 *dxb = static_cast<bf16 *>(dx);
    if (tile_dx2_fits<14, 14>(q.B, q.OH, q.OW, q.Cout, q.Cin, dy, wp, dx)) {
      launch_tile_dx2<14, 14>(dyb, wp, dxb, q.B, q.OH, q.Cout, q.Cin, d.tb.off, s);
      return true;
    }
    if (tile_dx2_fits<28, 7>(q.B, q.OH, q.OW, q.Cout, q.Cin, dy, wp, dx)) {
      launch_tile_dx2<28, 7>(dyb, wp, dxb, q.B, q.OH, q.Cout, q.Cin, d.tb.off, s);
      return true;
    }
  }
  const Scratch rest{static_cast<char *>(scr.ptr) + d.gemm_off, scr.bytes - d.gemm_off};
  for (int a = 0; a < q.SH; ++a)
    for (int c = 0; c < q.SW; ++c) {
      if (d.ah[a].T == 0 || d.aw[c].T == 0 || d.ah[a].U == 0 || d.aw[c].U == 0) continue;
      GemmParams p = dx_phase_gemm(d, a, c, dy, wp, dx, q);
      launch_gemm_mfma<false, kAConvVec>(p, TEENY_ACT_NONE, s, rest);
    }
  return true;
}

// The MFMA form of bf16 NHWC dx: the stride-1 conv it becomes and its scratch.
struct DxPlan {
  bool ok = false;
  ConvGeo g2;            // dy (or spread dy) -> dx
  bool spread = false;
  int HD = 0, WD = 0;
  size_t wt_bytes = 0, dyd_off = 0, gemm_off = 0;
};

static DxPlan dx_plan(const ConvGeo &q) {
  DxPlan d;
  if (q.G != 1 || q.PH > q.KH - 1 || q.PW > q.KW - 1 || q.Cout % 8 != 0) return d;
  d.spread = q.SH > 1 || q.SW > 1;
  d.HD = d.spread ? (q.OH - 1) * q.SH + 1 + (q.H + 2 * q.PH - q.KH) % q.SH : q.OH;
  d.WD = d.spread ? (q.OW - 1) * q.SW + 1 + (q.W + 2 * q.PW - q.KW) % q.SW : q.OW;
  teeny_conv2d_params p2{q.KH, q.KW, 1, 1, q.KH - 1 - q.PH, q.KW - 1 - q.PW, 1, TEENY_ACT_NONE};
  if (make_geo(q.B, q.Cout, q.Cin, d.HD, d.WD, q.H, q.W, &p2, TEENY_NHWC, &d.g2, "conv2d_backward_dx") != TEENY_OK)
    return d;
  if (conv_path<false>(d.g2) == kConvNoMfma) return d;
  d.ok = true;
  d.wt_bytes = static_cast<size_t>(q.Cout) * q.KH * q.KW * q.Cin * sizeof(bf16);
  d.dyd_off = round256(d.wt_bytes);
  d.gemm_off = d.dyd_off + (d.spread ? round256(static_cast<size_t>(q.B) * d.HD * d.WD * q.Cout * sizeof(bf16)) : 0);
  return d;
}

static size_t dx_scratch_bytes(const ConvGeo &q) {
  if (dx_phase_plan(q).ok) return dx_phase_scratch_bytes(q);
  const DxPlan d = dx_plan(q);
  return d.ok ? d.gemm_off + conv_scratch_bytes<false>(d.g2) : 0;
}

// bf16 NHWC dx on the MFMA path; false (nothing launched) if it does not apply.
static bool conv_dx_mfma(const void *dy, const void *w, void *dx, const ConvGeo &q, hipStream_t s, Scratch scr) {
  if (dx_phase_plan(q).ok) return conv_dx_phases(dy, w, dx, q, s, scr);
  const DxPlan d = dx_plan(q);
  if (!d.ok || scr.ptr == nullptr || scr.bytes < d.gemm_off || !aligned(dy, 16) || !aligned(w, 16)) return false;
  char *base = static_cast<char *>(scr.ptr);
  bf16 *wt = reinterpret_cast<bf16 *>(base);
  const int64_t nw = static_cast<int64_t>(q.Cout) * q.KH * q.KW * q.Cin;
  if (tap_transpose_ok(q, w, wt)) {
    // source tap (kh, kw) lands at the flipped tap (KH-1-kh, KW-1-kw) of wt [C_IN, KH, KW, C_OUT]
    TapMap m{};
    for (int kh = 0; kh < q.KH; ++kh)
      for (int kw = 0; kw < q.KW; ++kw) {
        m.D[kh * q.KW + kw] = static_cast<int64_t>((q.KH - 1 - kh) * q.KW + (q.KW - 1 - kw)) * q.Cout;
        m.R[kh * q.KW + kw] = q.KH * q.KW * q.Cout;
      }
    launch_tap_transpose(static_cast<const bf16 *>(w), wt, q, m, s);
  } else {
    hipLaunchKernelGGL(conv_bwd_flip_weights, dim3(static_cast<unsigned>(cdiv(nw, 256))), dim3(256), 0, s,
                       static_cast<const bf16 *>(w), wt, q.Cout, q.KH, q.KW, q.Cin);
  }
  const void *src = dy;
  if (d.spread) {
    bf16 *dyd = reinterpret_cast<bf16 *>(base + d.dyd_off);
    const int64_t nc = static_cast<int64_t>(q.B) * d.HD * d.WD * (q.Cout / 8);
    hipLaunchKernelGGL(conv_bwd_spread, dim3(static_cast<unsigned>(cdiv(nc, 256))), dim3(256), 0, s,
                       static_cast<const bf16 *>(dy), dyd, q.B, q.OH, q.OW, q.Cout, d.HD, d.WD, q.SH, q.SW);
    src = dyd;
  }
  const Scratch rest{base + d.gemm_off, scr.bytes - d.gemm_off};
  if (try_conv_mfma<false>(src, wt, nullptr, nullptr, nullptr, dx, d.g2, TEENY_ACT_NONE, s, rest)) return true;
  // the GEMM declined (alignment): the direct kernel reads the caller's buffers
  return false;
}

template <typename T>
static void launch_dx_direct(const void *dy, const void *w, void *dx, const ConvGeo &q, bool nhwc, hipStream_t s) {
  const int64_t total = static_cast<int64_t>(q.B) * q.Cin * q.H * q.W;
  hipLaunchKernelGGL((conv_bwd_dx_direct<T>), dim3(static_cast<unsigned>(cdiv(total, 256))), dim3(256), 0, s,
                     static_cast<const T *>(dy), static_cast<const T *>(w), static_cast<T *>(dx), q, nhwc ? 1 : 0);
}

template <typename T>
static void launch_dw_direct(const void *dy, const void *x, void *dw, const ConvGeo &q, hipStream_t s) {
  const int64_t n = static_cast<int64_t>(q.Cout) * (q.Cin / q.G) * q.KH * q.KW;
  hipLaunchKernelGGL((conv_bwd_dw_direct<T>), dim3(static_cast<unsigned>(n)), dim3(256), 0, s,
                     static_cast<const T *>(dy), static_cast<const T *>(x), static_cast<T *>(dw), q);
}

// ── bf16 NHWC dw on the matrix cores ──
// dw[co, (kh, kw, ci)] = sum over pixels p = (b, oh, ow) of dy[p, co] *
// x[b, oh*SH - PH + kh, ow*SW - PW + kw, ci]: a GEMM with M = C_OUT,
// N = KH*KW*C_IN and the reduction over the B*OH*OW pixels.  Both operands
// arrive pixel-major (rows of dy, gathered rows of x), so stages of 64
// pixels x 128 columns of each are moved to LDS by LDS-DMA (padding taps,
// rows past the last pixel and columns past the edge read as zeros through
// the buffer extent) and both MFMA operands come out of LDS through
// transposing reads.  Workgroup tile 128 x 128, four waves of 64 x 64.  The
// pixel range is split over workgroups; with more than one split each
// writes fp32 partials to the stream workspace and a second kernel adds them
// in split order (deterministic).
constexpr int kDwTile = 128, kDwStage = 64;

struct DwPlan {
  bool ok = false;
  int tiles_m = 0, tiles_n = 0, splits = 1, stages_per_split = 0;
  size_t part_bytes = 0;  // workspace for splits > 1
};

// `workspace`: bytes the caller's stream offers (the split count shrinks to fit).
static DwPlan dw_plan(const ConvGeo &q, size_t workspace) {
  DwPlan d;
  if (q.G != 1 || q.Cin % 8 != 0 || q.Cout % 8 != 0 || q.B == 0) return d;
  const int64_t P = static_cast<int64_t>(q.B) * q.OH * q.OW;
  const int64_t M = q.Cout, N = static_cast<int64_t>(q.KH) * q.KW * q.Cin;
  // 32-bit buffer offsets into dy and x
  if (P * M * 2 > 0x7fffff00LL || static_cast<int64_t>(q.B) * q.H * q.W * q.Cin * 2 > 0x7fffff00LL) return d;
  d.tiles_m = static_cast<int>(cdiv(M, kDwTile));
  d.tiles_n = static_cast<int>(cdiv(N, kDwTile));
  const int64_t tiles = static_cast<int64_t>(d.tiles_m) * d.tiles_n, stages = cdiv(P, kDwStage);
  int64_t splits = cdiv(2 * static_cast<int64_t>(device_cu_count()), tiles);  // about two workgroups per CU
  splits = std::min<int64_t>(splits, std::max<int64_t>(1, stages / 4));       // at least 4 stages per split
  while (splits > 1 && static_cast<size_t>(splits) * M * N * 4 > workspace) --splits;
  d.stages_per_split = static_cast<int>(cdiv(stages, splits));
  d.splits = static_cast<int>(cdiv(stages, d.stages_per_split));  // no empty split
  d.part_bytes = d.splits > 1 ? static_cast<size_t>(d.splits) * M * N * 4 : 0;
  d.ok = tiles * d.splits <= 0x7fffffff;
  return d;
}

// The split count the kernel would like (what the workspace-size query reports).
static size_t dw_scratch_bytes(const ConvGeo &q) { return dw_plan(q, static_cast<size_t>(1) << 26).part_bytes; }

template <bool PART>
__global__ __launch_bounds__(256, 2) void conv_dw_mfma(const bf16 *__restrict__ dy, const bf16 *__restrict__ x,
                                                       bf16 *__restrict__ dw, float *__restrict__ part, ConvGeo q,
                                                       int tiles_m, int tiles_n, int stages_per_split, int P) {
  constexpr int NT = 256, TILE = kDwStage * kDwTile;
  __shared__ __attribute__((aligned(16))) bf16 abuf[2][TILE], bbuf[2][TILE];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, c = lane & 31;
  const int ntiles = tiles_m * tiles_n;
  // the tiles of one split (same pixels of dy and x) are consecutive ids: one XCD's L2
  const int id = xcd_remap(blockIdx.x, gridDim.x);
  const int split = id / ntiles, t = id % ntiles;
  const int co0 = (t / tiles_n) * kDwTile, n0 = (t % tiles_n) * kDwTile;
  const int M = q.Cout, N = q.KH * q.KW * q.Cin;
  const int wm = w >> 1, wn = w & 1;
  const int st0 = split * stages_per_split;
  const int nst = min(stages_per_split, (P + kDwStage - 1) / kDwStage - st0);
  const __amdgpu_buffer_rsrc_t dys = buffer_rsrc(dy, P * M * 2);
  const __amdgpu_buffer_rsrc_t xs = buffer_rsrc(x, q.B * q.H * q.W * q.Cin * 2);
  // LDS-DMA slot u = 256 i + tid: stage row 16 i + tid / 16, chunk position
  // tid % 16, holding logical 16-byte chunk `chunk` (the row swizzle depends
  // on row % 16 only, so it is the same in every round)
  const int lrow = tid >> 4;
  const int chunk = (tid & 15) ^ bswz<128>(lrow);
  const int a_col = co0 + 8 * chunk;
  const bool a_ok = a_col < M;
  const int nb = n0 + 8 * chunk;
  const bool b_ok = nb < N;
  const int tap = nb / q.Cin, ci = nb % q.Cin;  // C_IN % 8 == 0: a chunk never straddles two taps
  const int kh = tap / q.KW, kw = tap % q.KW;
  auto issue = [&](int s, int b) __attribute__((always_inline)) {
    const int p0 = (st0 + s) * kDwStage;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int p = p0 + 16 * i + lrow;
      int aoff = kOffNone, boff = kOffNone;
      if (p < P) {
        if (a_ok) aoff = (p * M + a_col) * 2;
        if (b_ok) {
          const int ow = p % q.OW, r = p / q.OW;
          const int oh = r % q.OH, bb = r / q.OH;
          const int ih = oh * q.SH - q.PH + kh, iw = ow * q.SW - q.PW + kw;
          if (ih >= 0 && ih < q.H && iw >= 0 && iw < q.W) boff = (((bb * q.H + ih) * q.W + iw) * q.Cin + ci) * 2;
        }
      }
      buffer_lds_dma16(dys, aoff, __builtin_amdgcn_readfirstlane(lds_address(abuf[b] + (NT * i + 64 * w) * 8)));
      buffer_lds_dma16(xs, boff, __builtin_amdgcn_readfirstlane(lds_address(bbuf[b] + (NT * i + 64 * w) * 8)));
    }
  };
  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = zero16();
  if (nst > 0) {
    issue(0, 0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  }
  for (int s = 0; s < nst; ++s) {
    const int b = s & 1;
    if (s + 1 < nst) issue(s + 1, b ^ 1);
#pragma unroll
    for (int kk = 0; kk < kDwStage / 16; ++kk) {
      bf16x8 af[2], bfr[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) af[i] = frag_tr<128>(abuf[b], 16 * kk, 2 * wm + i, lane);
#pragma unroll
      for (int j = 0; j < 2; ++j) bfr[j] = frag_tr<128>(bbuf[b], 16 * kk, 2 * wn + j, lane);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = mfma32x32x16(af[i], bfr[j], acc[i][j]);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  }
  // lane (g, c) holds column n0 + 64 wn + 32 j + c, rows co0 + 64 wm + 32 i + mfma32_row(v, g)
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = n0 + 64 * wn + 32 * j + c;
      if (n >= N) continue;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int m = co0 + 64 * wm + 32 * i + mfma32_row(v, g);
        if (m >= M) continue;
        // partials by non-temporal stores (1x1 512 -> 2048 dw 27.2 -> 24.7 us,
        // 3x3 128 -> 128 40.1 -> 39.3 us)
        if constexpr (PART) __builtin_nontemporal_store(acc[i][j][v], part + (static_cast<int64_t>(split) * M + m) * N + n);
        else dw[static_cast<int64_t>(m) * N + n] = static_cast<bf16>(acc[i][j][v]);
      }
    }
}

// dw = sum of the splits' fp32 partials, in split order, rounded to bf16.
__global__ __launch_bounds__(256) void conv_dw_reduce_seq(const float *__restrict__ part, bf16 *__restrict__ dw,
                                                          int splits, int64_t mn) {
  const int64_t i = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 4;
  if (i >= mn) return;
  auto at = [&](int k) { return __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(part + k * mn + i)); };
  f32x4 s = at(0);
  int k = 1;
  // eight splits' loads in flight, added in split order (the sum is the
  // same, bit for bit, as one load and add at a time)
  for (; k + 8 <= splits; k += 8) {
    f32x4 t[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) t[u] = at(k + u);
#pragma unroll
    for (int u = 0; u < 8; ++u) s += t[u];
  }
  for (; k < splits; ++k) s += at(k);
  bf16x4 o;
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = static_cast<bf16>(s[e]);
  *reinterpret_cast<bf16x4 *>(dw + i) = o;
}

// dw = sum of the splits' fp32 partials, rounded to bf16, in a fixed order:
// each output quad (4 consecutive floats) has `sub` threads (a power of two,
// at most 8, the least that leaves each thread at most eight splits), thread
// j summing splits [j per, (j + 1) per) in order with its loads issued
// together, and the `sub` sums are added in thread order through LDS.  (One
// thread per quad walking every split ran the 3x3 128 -> 128 layer's 57
// splits over 144 workgroups: 39.5 against 36.9 us for its dw; with at
// most eight splits that form, conv_dw_reduce_seq, is kept: the 1x1
// 512 -> 2048 layer's 7 splits 24.8 against 26.3 us.)
__global__ __launch_bounds__(256) void conv_dw_reduce(const float *__restrict__ part, bf16 *__restrict__ dw,
                                                      int splits, int64_t mn, int sub) {
  __shared__ f32x4 red[256];
  const int t = threadIdx.x, j = t & (sub - 1), qi = t / sub;
  const int64_t i = (static_cast<int64_t>(blockIdx.x) * (256 / sub) + qi) * 4;
  const int per = (splits + sub - 1) / sub;
  const int k0 = min(splits, j * per), k1 = min(splits, k0 + per);
  f32x4 s = {0.0f, 0.0f, 0.0f, 0.0f};
  if (i < mn) {
    auto at = [&](int k) { return __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(part + k * mn + i)); };
    for (int k = k0; k < k1; k += 8) {
      f32x4 v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (k + u < k1) v[u] = at(k + u);
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (k + u < k1) s += v[u];
    }
  }
  red[t] = s;
  __syncthreads();
  if (j == 0 && i < mn) {
    f32x4 tot = red[t];
    for (int m = 1; m < sub; ++m) tot += red[t + m];
    bf16x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = static_cast<bf16>(tot[e]);
    *reinterpret_cast<bf16x4 *>(dw + i) = o;
  }
}

// bf16 NHWC dw on the MFMA path; false (nothing launched) if it does not apply.
static bool conv_dw_mfma_launch(const void *dy, const void *x, void *dw, const ConvGeo &q, hipStream_t s,
                                Scratch scr) {
  if (!aligned(dy, 16) || !aligned(x, 16) || !aligned(dw, 8)) return false;
  const DwPlan d = dw_plan(q, scr.ptr != nullptr ? scr.bytes : 0);
  if (!d.ok) return false;
  const int P = q.B * q.OH * q.OW;
  const dim3 grid(static_cast<unsigned>(d.tiles_m * d.tiles_n * d.splits));
  if (d.splits > 1) {
    float *part = static_cast<float *>(scr.ptr);
    hipLaunchKernelGGL(conv_dw_mfma<true>, grid, dim3(256), 0, s, static_cast<const bf16 *>(dy),
                       static_cast<const bf16 *>(x), static_cast<bf16 *>(dw), part, q, d.tiles_m, d.tiles_n,
                       d.stages_per_split, P);
    const int64_t mn = static_cast<int64_t>(q.Cout) * q.KH * q.KW * q.Cin;
    int sub = 1;
    while (sub < 8 && cdiv(d.splits, sub) > 8) sub *= 2;
    if (sub == 1)
      hipLaunchKernelGGL(conv_dw_reduce_seq, dim3(static_cast<unsigned>(cdiv(mn / 4, 256))), dim3(256), 0, s, part,
                         static_cast<bf16 *>(dw), d.splits, mn);
    else
      hipLaunchKernelGGL(conv_dw_reduce, dim3(static_cast<unsigned>(cdiv(mn / 4, 256 / sub))), dim3(256), 0, s, part,
                         static_cast<bf16 *>(dw), d.splits, mn, sub);
  } else {
    hipLaunchKernelGGL(conv_dw_mfma<false>, grid, dim3(256), 0, s, static_cast<const bf16 *>(dy),
                       static_cast<const bf16 *>(x), static_cast<bf16 *>(dw), nullptr, q, d.tiles_m, d.tiles_n,
                       d.stages_per_split, P);
  }
  return true;
}

static teeny_status conv_bwd_entry(const void *dy, const void *x, const void *w, void *dx, void *dw, int64_t B,
                                   int64_t Cin, int64_t Cout, int64_t H, int64_t W, int64_t OH, int64_t OW,
                                   const teeny_conv2d_params *prm, teeny_dtype dtype, teeny_layout layout,
                                   teeny_stream stream, const char *name) {
  ConvGeo q;
  teeny_status st = make_geo(B, Cin, Cout, H, W, OH, OW, prm, layout, &q, name);
  if (st != TEENY_OK) return st;
  TEENY_REQUIRE(dtype == TEENY_F32 || dtype == TEENY_BF16, TEENY_ERR_UNSUPPORTED_DTYPE,
                std::string(name) + ": dtype must be F32 or BF16");
  TEENY_REQUIRE(static_cast<int64_t>(Cout) * (Cin / prm->groups) * prm->KH * prm->KW <= 0x7fffffff,
                TEENY_ERR_SHAPE_MISMATCH, std::string(name) + ": weight too large");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (B == 0) {  // an empty batch: dx is empty, dw = 0 (a sum over no pixels)
    if (dw == nullptr) return TEENY_OK;
    if (dtype == TEENY_F32) launch_dw_direct<float>(dy, x, dw, q, s);
    else launch_dw_direct<bf16>(dy, x, dw, q, s);
    return after_launch(name, s);
  }
  TEENY_REQUIRE(dy != nullptr && (dx == nullptr || w != nullptr) && (dw == nullptr || x != nullptr),
                TEENY_ERR_NULL_POINTER, std::string(name) + ": dy/w/x");
  const bool nhwc = layout == TEENY_NHWC;
  if (dx != nullptr) {
    if (!(dtype == TEENY_BF16 && nhwc && conv_dx_mfma(dy, w, dx, q, s, stream_scratch(s)))) {
      if (dtype == TEENY_F32) launch_dx_direct<float>(dy, w, dx, q, nhwc, s);
      else launch_dx_direct<bf16>(dy, w, dx, q, nhwc, s);
    }
    st = after_launch(name, s);
    if (st != TEENY_OK) return st;
  }
  if (dw != nullptr) {
    if (!(dtype == TEENY_BF16 && nhwc && conv_dw_mfma_launch(dy, x, dw, q, s, stream_scratch(s)))) {
      if (dtype == TEENY_F32) launch_dw_direct<float>(dy, x, dw, q, s);
      else launch_dw_direct<bf16>(dy, x, dw, q, s);
    }
    st = after_launch(name, s);
  }
  return st;
}

// ── the no-allocation variant's scratch ─────────────────────────────────
// A file-scope device array serves as the scratch of
// teeny_conv2d_bias_forward_noalloc.  Each GPU that loads this library holds
// its own copy (at its own address) until the process ends.  Its host-side
// name is not a device address: the device address comes from
// hipGetSymbolAddress, once per device on the entry point's first call there.
constexpr size_t kStaticScratchBytes = size_t(32) << 20;
static __device__ __align__(256) char scratch[kStaticScratchBytes];
static std::mutex g_scratch_addr_mu;
static void *g_scratch_addr[64];

static teeny_status static_scratch(Scratch *out, const char *name) {
  int dev = 0;
  TEENY_CHECK_HIP(hipGetDevice(&dev));
  TEENY_REQUIRE(dev >= 0 && dev < 64, TEENY_ERR_UNSUPPORTED, std::string(name) + ": device ordinal >= 64");
  std::lock_guard<std::mutex> lock(g_scratch_addr_mu);
  if (g_scratch_addr[dev] == nullptr) {
    void *ptr = nullptr;
    TEENY_CHECK_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
    TEENY_REQUIRE(ptr != nullptr && aligned(ptr, 256), TEENY_ERR_HIP,
                  std::string(name) + ": static scratch has no usable device address");
    g_scratch_addr[dev] = ptr;
  }
  *out = Scratch{g_scratch_addr[dev], kStaticScratchBytes};
  return TEENY_OK;
}

}  // namespace teeny

using namespace teeny;

extern "C" {

teeny_status teeny_conv2d_forward(const void *x, const void *w, void *y, int64_t B, int64_t C_IN,
                                  int64_t C_OUT, int64_t H, int64_t W, int64_t OH, int64_t OW,
                                  const teeny_conv2d_params *params, teeny_dtype dtype,
                                  teeny_layout layout, teeny_stream stream) {
  return conv_entry(x, w, nullptr, y, B, C_IN, C_OUT, H, W, OH, OW, params, dtype, layout, stream,
                    "conv2d_forward");
}

teeny_status teeny_conv2d_bias_forward(const void *x, const void *w, const void *bias, void *y,
                                       int64_t B, int64_t C_IN, int64_t C_OUT, int64_t H,
                                       int64_t W, int64_t OH, int64_t OW,
                                       const teeny_conv2d_params *params, teeny_dtype dtype,
                                       teeny_layout layout, teeny_stream stream) {
  TEENY_REQUIRE(bias != nullptr, TEENY_ERR_NULL_POINTER, "conv2d_bias_forward: bias");
  return conv_entry(x, w, bias, y, B, C_IN, C_OUT, H, W, OH, OW, params, dtype, layout, stream,
                    "conv2d_bias_forward");
}

teeny_status teeny_conv2d_bn_act_forward(const void *x, const void *w, const float *bn_scale, const float *bn_shift,
                                        void *y, int64_t B, int64_t C_IN, int64_t C_OUT, int64_t H, int64_t W,
                                        int64_t OH, int64_t OW, const int64_t *y_strides,
                                        const teeny_conv2d_params *params, teeny_dtype dtype, teeny_layout layout,
                                        teeny_stream stream) {
  return conv_bn_entry(x, w, bn_scale, bn_shift, y, B, C_IN, C_OUT, H, W, OH, OW, y_strides, params, dtype, layout,
                       stream, "conv2d_bn_act_forward");
}

teeny_status teeny_conv2d_bias_forward_noalloc(const void *x, const void *w, const void *bias, void *y,
                                               int64_t B, int64_t C_IN, int64_t C_OUT, int64_t H,
                                               int64_t W, int64_t OH, int64_t OW,
                                               const teeny_conv2d_params *params, teeny_dtype dtype,
                                               teeny_layout layout, teeny_stream stream) {
  const char *name = "conv2d_bias_forward_noalloc";
  ConvGeo q;
  teeny_status st = make_geo(B, C_IN, C_OUT, H, W, OH, OW, params, layout, &q, name);
  if (st != TEENY_OK) return st;
  TEENY_REQUIRE(dtype == TEENY_F32 || dtype == TEENY_BF16, TEENY_ERR_UNSUPPORTED_DTYPE,
                std::string(name) + ": dtype must be F32 or BF16");
  if (B == 0) return TEENY_OK;
  TEENY_REQUIRE(x != nullptr && w != nullptr && bias != nullptr && y != nullptr, TEENY_ERR_NULL_POINTER,
                std::string(name) + ": x/w/bias/y");
  const size_t need = (dtype == TEENY_BF16 && layout == TEENY_NHWC) ? conv_scratch_bytes<false>(q) : 0;
  TEENY_REQUIRE(need <= kStaticScratchBytes, TEENY_ERR_UNSUPPORTED,
                std::string(name) + ": this shape's plan needs " + std::to_string(need) +
                    " bytes of scratch, more than the " + std::to_string(kStaticScratchBytes) +
                    " bytes of static scratch; use conv2d_bias_forward with a stream workspace");
  Scratch scr;
  st = static_scratch(&scr, name);
  if (st != TEENY_OK) return st;
  return conv_entry(x, w, bias, y, B, C_IN, C_OUT, H, W, OH, OW, params, dtype, layout, stream, name, &scr);
}

teeny_status teeny_w8a16_conv2d_forward(const void *x, const int8_t *qweight, const float *scale,
                                        const float *bias, void *y, int64_t B, int64_t C_IN,
                                        int64_t C_OUT, int64_t H, int64_t W, int64_t OH,
                                        int64_t OW, const teeny_conv2d_params *params,
                                        teeny_stream stream) {
  const char *name = "w8a16_conv2d_forward";
  ConvGeo q;
  teeny_status st = make_geo(B, C_IN, C_OUT, H, W, OH, OW, params, TEENY_NHWC, &q, name);
  if (st != TEENY_OK) return st;
  if (B == 0) return TEENY_OK;
  TEENY_REQUIRE(x != nullptr && qweight != nullptr && scale != nullptr && y != nullptr,
                TEENY_ERR_NULL_POINTER, "w8a16_conv2d_forward: x/qweight/scale/y");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (!try_conv_mfma<true>(x, qweight, scale, bias, nullptr, y, q, params->act, s, stream_scratch(s))) {
    launch_direct<bf16, int8_t>(static_cast<const bf16 *>(x), qweight, scale, nullptr, bias,
                                static_cast<bf16 *>(y), q, params->act, s);
  }
  return after_launch(name, s);
}

teeny_status teeny_conv2d_backward_dx(const void *dy, const void *w, void *dx, int64_t B, int64_t C_IN,
                                      int64_t C_OUT, int64_t H, int64_t W, int64_t OH, int64_t OW,
                                      const teeny_conv2d_params *params, teeny_dtype dtype, teeny_layout layout,
                                      teeny_stream stream) {
  TEENY_REQUIRE(dx != nullptr, TEENY_ERR_NULL_POINTER, "conv2d_backward_dx: dx");
  return conv_bwd_entry(dy, nullptr, w, dx, nullptr, B, C_IN, C_OUT, H, W, OH, OW, params, dtype, layout, stream,
                        "conv2d_backward_dx");
}

teeny_status teeny_conv2d_backward_dw(const void *dy, const void *x, void *dw, int64_t B, int64_t C_IN,
                                      int64_t C_OUT, int64_t H, int64_t W, int64_t OH, int64_t OW,
                                      const teeny_conv2d_params *params, teeny_dtype dtype, teeny_layout layout,
                                      teeny_stream stream) {
  TEENY_REQUIRE(dw != nullptr, TEENY_ERR_NULL_POINTER, "conv2d_backward_dw: dw");
  return conv_bwd_entry(dy, x, nullptr, nullptr, dw, B, C_IN, C_OUT, H, W, OH, OW, params, dtype, layout, stream,
                        "conv2d_backward_dw");
}

teeny_status teeny_conv2d_backward(const void *dy, const void *x, const void *w, void *dx, void *dw, int64_t B,
                                   int64_t C_IN, int64_t C_OUT, int64_t H, int64_t W, int64_t OH, int64_t OW,
                                   const teeny_conv2d_params *params, teeny_dtype dtype, teeny_layout layout,
                                   teeny_stream stream) {
  TEENY_REQUIRE(dx != nullptr && dw != nullptr, TEENY_ERR_NULL_POINTER, "conv2d_backward: dx/dw");
  return conv_bwd_entry(dy, x, w, dx, dw, B, C_IN, C_OUT, H, W, OH, OW, params, dtype, layout, stream,
                        "conv2d_backward");
}

teeny_status teeny_conv2d_backward_workspace_size(int64_t B, int64_t C_IN, int64_t C_OUT, int64_t H, int64_t W,
                                                  int64_t OH, int64_t OW, const teeny_conv2d_params *params,
                                                  teeny_dtype dtype, teeny_layout layout, size_t *bytes) {
  TEENY_REQUIRE(bytes != nullptr, TEENY_ERR_NULL_POINTER, "conv2d_backward_workspace_size: bytes");
  *bytes = 0;
  ConvGeo q;
  teeny_status st = make_geo(B, C_IN, C_OUT, H, W, OH, OW, params, layout, &q, "conv2d_backward_workspace_size");
  if (st != TEENY_OK) return st;
  TEENY_REQUIRE(dtype == TEENY_F32 || dtype == TEENY_BF16, TEENY_ERR_UNSUPPORTED_DTYPE,
                "conv2d_backward_workspace_size: dtype must be F32 or BF16");
  if (B > 0 && dtype == TEENY_BF16 && layout == TEENY_NHWC) *bytes = std::max(dx_scratch_bytes(q), dw_scratch_bytes(q));
  return TEENY_OK;
}

teeny_status teeny_conv2d_workspace_size(int64_t B, int64_t C_IN, int64_t C_OUT, int64_t H, int64_t W,
                                         int64_t OH, int64_t OW, const teeny_conv2d_params *params,
                                         teeny_dtype dtype, teeny_layout layout, size_t *bytes) {
  const char *name = "conv2d_workspace_size";
  TEENY_REQUIRE(bytes != nullptr, TEENY_ERR_NULL_POINTER, "conv2d_workspace_size: bytes");
  *bytes = 0;
  ConvGeo q;
  teeny_status st = make_geo(B, C_IN, C_OUT, H, W, OH, OW, params, layout, &q, name);
  if (st != TEENY_OK) return st;
  if (B == 0 || layout != TEENY_NHWC) return TEENY_OK;
  if (dtype == TEENY_BF16) *bytes = conv_scratch_bytes<false>(q);
  else if (dtype == TEENY_I8) *bytes = conv_scratch_bytes<true>(q);
  else TEENY_REQUIRE(dtype == TEENY_F32, TEENY_ERR_UNSUPPORTED_DTYPE, "conv2d_workspace_size: dtype");
  return TEENY_OK;
}

}  // extern "C"
