// Linear layers: linear_forward (fp32 / bf16) and the W8A16 int8-weight GEMM.
//
// Reference: linear_forward, kernels/teeny-kernels/src/nn/mlp/linear.rs:20-116
// (y = x W^T (+ b), x [M,K], W [N,K], arbitrary strides, GROUP_M-swizzled
// BLOCK_M x BLOCK_N tiles, TF32 tl.dot), RuntimeOp :250-320.  The W8A16
// variant has no reference kernel: it is linear_forward applied to the
// weights that teeny-quant's dequantize_affine reconstructs
// (utilities/teeny-quant/src/quant/affine.rs:151-161) from per-output-channel
// symmetric int8 (granularity PerChannel{axis: 0}, groups.rs:82-87).
//
// bf16 and int8 weights run on the MFMA core (gemm_core.hpp) whenever the
// operands are K-contiguous and 16-byte aligned; anything else (fp32, odd
// strides, ragged K for int8) runs gemm_generic: a 64 x 64 LDS-tiled fp32 FMA
// kernel that accumulates each output in k order.
#include "gemm_core.hpp"

namespace teeny {

template <typename T> __device__ __forceinline__ float ld_f32(const T *p, int64_t i) {
  return to_f32(p[i]);
}
template <> __device__ __forceinline__ float ld_f32<int8_t>(const int8_t *p, int64_t i) {
  return static_cast<float>(p[i]);
}

// C[m,n] = act(scale[n] * sum_k A[m,k] B[n,k] + bias[n]); bias typed TC
// (linear_forward) or fp32 (W8A16).  16 x 16 threads, 4 x 4 outputs each.
template <typename TA, typename TB, typename TC, int ACT>
__global__ __launch_bounds__(256) void gemm_generic(const TA *__restrict__ A, int64_t sam,
                                                    int64_t sak, const TB *__restrict__ B,
                                                    int64_t sbn, int64_t sbk, TC *__restrict__ C,
                                                    int64_t scm, int64_t scn,
                                                    const float *__restrict__ scale,
                                                    const TC *__restrict__ bias_t,
                                                    const float *__restrict__ bias_f, int M, int N,
                                                    int K) {
  constexpr int T = 64, KC = 16;
  __shared__ float as[KC][T + 1];
  __shared__ float bs[KC][T + 1];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int m0 = blockIdx.y * T, n0 = blockIdx.x * T;
  float acc[4][4] = {};
  for (int k0 = 0; k0 < K; k0 += KC) {
    for (int i = threadIdx.x; i < KC * T; i += 256) {
      const int kk = i % KC, r = i / KC;
      const int m = m0 + r, n = n0 + r, k = k0 + kk;
      as[kk][r] = (m < M && k < K) ? ld_f32(A, m * sam + k * sak) : 0.0f;
      bs[kk][r] = (n < N && k < K) ? ld_f32(B, n * sbn + k * sbk) : 0.0f;
    }
    __syncthreads();
    const int kn = min(KC, K - k0);
    for (int kk = 0; kk < kn; ++kk) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] += as[kk][ty + 16 * i] * bs[kk][tx + 16 * j];
    }
    __syncthreads();
  }
  constexpr bool fast = !std::is_same<TC, float>::value;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = m0 + ty + 16 * i;
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + tx + 16 * j;
      if (n >= N) continue;
      float r = acc[i][j];
      if (scale != nullptr) r *= scale[n];
      if (bias_t != nullptr) r = r + to_f32(bias_t[n]);
      if (bias_f != nullptr) r = r + bias_f[n];
      C[m * scm + n * scn] = from_f32<TC>(apply_act<ACT, fast>(r));
    }
  }
}

template <typename TA, typename TB, typename TC>
static teeny_status launch_generic(const TA *A, int64_t sam, int64_t sak, const TB *B, int64_t sbn,
                                   int64_t sbk, TC *C, int64_t scm, int64_t scn,
                                   const float *scale, const TC *bias_t, const float *bias_f,
                                   int64_t M, int64_t N, int64_t K, int act, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(cdiv(N, 64)), static_cast<unsigned>(cdiv(M, 64)));
  TEENY_REQUIRE(grid.y <= 65535, TEENY_ERR_SHAPE_MISMATCH, "gemm: M too large for generic path");
#define TEENY_GEMM_GENERIC(ACTV)                                                                   \
  hipLaunchKernelGGL((gemm_generic<TA, TB, TC, ACTV>), grid, dim3(256), 0, s, A, sam, sak, B, sbn, \
                     sbk, C, scm, scn, scale, bias_t, bias_f, static_cast<int>(M),                 \
                     static_cast<int>(N), static_cast<int>(K))
  switch (act) {
    case TEENY_ACT_NONE: TEENY_GEMM_GENERIC(TEENY_ACT_NONE); break;
    case TEENY_ACT_RELU: TEENY_GEMM_GENERIC(TEENY_ACT_RELU); break;
    case TEENY_ACT_GELU_TANH: TEENY_GEMM_GENERIC(TEENY_ACT_GELU_TANH); break;
    case TEENY_ACT_SILU: TEENY_GEMM_GENERIC(TEENY_ACT_SILU); break;
    default: return fail(TEENY_ERR_INVALID_ARGUMENT, "gemm: unknown activation");
  }
#undef TEENY_GEMM_GENERIC
  return TEENY_OK;
}

// db[n] = sum_m dy[m, n] in m order, fp32 (linear_backward's bias gradient).
// 64 threads per block: one column each, consecutive columns per wave.
template <typename T>
__global__ __launch_bounds__(64) void linear_bwd_db(const T *__restrict__ dy, int64_t sm, int64_t sn,
                                                    T *__restrict__ db, int64_t sdb, int M, int N) {
  const int n = blockIdx.x * 64 + threadIdx.x;
  if (n >= N) return;
  float acc = 0.0f;
  const T *col = dy + n * sn;
  for (int m = 0; m < M; ++m) acc += to_f32(col[m * sm]);
  db[n * sdb] = from_f32<T>(acc);
}

static GemmParams plain_params(const void *A, int64_t lda, const void *B, int64_t ldb, void *C,
                               int64_t ldc, const float *scale, const float *bias,
                               const bf16 *bias_bf16, int64_t M, int64_t N, int64_t K) {
  GemmParams p{};
  p.A = static_cast<const bf16 *>(A);
  p.lda = lda;
  p.B = B;
  p.ldb = ldb;
  p.C = static_cast<bf16 *>(C);
  p.ldc = ldc;
  p.scale = scale;
  p.bias = bias;
  p.bias_bf16 = bias_bf16;
  p.M = static_cast<int>(M);
  p.N = static_cast<int>(N);
  p.K = static_cast<int>(K);
  return p;
}

}  // namespace teeny

using namespace teeny;

extern "C" {

teeny_status teeny_linear_forward(const void *x, const void *w, const void *b, void *y, int64_t M,
                                  int64_t N, int64_t K, int64_t stride_xm, int64_t stride_xk,
                                  int64_t stride_wn, int64_t stride_wk, int64_t stride_ym,
                                  int64_t stride_yn, teeny_dtype dtype, teeny_stream stream) {
  TEENY_REQUIRE(M >= 0 && N >= 0 && K >= 0, TEENY_ERR_SHAPE_MISMATCH, "linear_forward: negative size");
  if (M == 0 || N == 0) return TEENY_OK;
  TEENY_REQUIRE(M <= 0x7fffffff && N <= 0x7fffffff && K <= 0x7fffffff, TEENY_ERR_SHAPE_MISMATCH,
                "linear_forward: size exceeds 2^31-1");
  TEENY_REQUIRE(y != nullptr && (K == 0 || (x != nullptr && w != nullptr)), TEENY_ERR_NULL_POINTER,
                "linear_forward: x/w/y");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == TEENY_F32) {
    teeny_status st = launch_generic<float, float, float>(
        static_cast<const float *>(x), stride_xm, stride_xk, static_cast<const float *>(w),
        stride_wn, stride_wk, static_cast<float *>(y), stride_ym, stride_yn, nullptr,
        static_cast<const float *>(b), nullptr, M, N, K, TEENY_ACT_NONE, s);
    if (st != TEENY_OK) return st;
    return after_launch("linear_forward", s);
  }
  if (dtype == TEENY_BF16) {
    const bool mfma_ok = stride_xk == 1 && stride_wk == 1 && stride_yn == 1 && stride_xm % 8 == 0 &&
                         stride_wn % 8 == 0 && aligned(x, 16) && aligned(w, 16) && K > 0;
    if (mfma_ok) {
      GemmParams p = plain_params(x, stride_xm, w, stride_wn, y, stride_ym, nullptr, nullptr,
                                  static_cast<const bf16 *>(b), M, N, K);
      launch_gemm_mfma<false, kAPlain>(p, TEENY_ACT_NONE, s, stream_scratch(s));
    } else {
      teeny_status st = launch_generic<bf16, bf16, bf16>(
          static_cast<const bf16 *>(x), stride_xm, stride_xk, static_cast<const bf16 *>(w),
          stride_wn, stride_wk, static_cast<bf16 *>(y), stride_ym, stride_yn, nullptr,
          static_cast<const bf16 *>(b), nullptr, M, N, K, TEENY_ACT_NONE, s);
      if (st != TEENY_OK) return st;
    }
    return after_launch("linear_forward", s);
  }
  return fail(TEENY_ERR_UNSUPPORTED_DTYPE, "linear_forward: dtype must be F32 or BF16");
}

teeny_status teeny_w8a16_linear_forward(const void *x, const int8_t *qweight, const float *scale,
                                        const float *bias, void *y, int64_t M, int64_t N,
                                        int64_t K, teeny_activation act, teeny_stream stream) {
  TEENY_REQUIRE(M >= 0 && N >= 0 && K >= 0, TEENY_ERR_SHAPE_MISMATCH,
                "w8a16_linear_forward: negative size");
  if (M == 0 || N == 0) return TEENY_OK;
  TEENY_REQUIRE(M <= 0x7fffffff && N <= 0x7fffffff && K <= 0x7fffffff, TEENY_ERR_SHAPE_MISMATCH,
                "w8a16_linear_forward: size exceeds 2^31-1");
  TEENY_REQUIRE(y != nullptr && scale != nullptr && (K == 0 || (x != nullptr && qweight != nullptr)),
                TEENY_ERR_NULL_POINTER, "w8a16_linear_forward: x/qweight/scale/y");
  TEENY_REQUIRE(act >= TEENY_ACT_NONE && act <= TEENY_ACT_SILU, TEENY_ERR_INVALID_ARGUMENT,
                "w8a16_linear_forward: unknown activation");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool mfma_ok = K > 0 && K % 16 == 0 && aligned(x, 16) && aligned(qweight, 16);
  if (mfma_ok) {
    GemmParams p = plain_params(x, K, qweight, K, y, N, scale, bias, nullptr, M, N, K);
    // int8 weights stay int8 up to the registers feeding the MFMA (no
    // dequantized copy in HBM)
    launch_gemm_mfma<true, kAPlain>(p, act, s, stream_scratch(s));
  } else {
    teeny_status st = launch_generic<bf16, int8_t, bf16>(
        static_cast<const bf16 *>(x), K, 1, qweight, K, 1, static_cast<bf16 *>(y), N, 1, scale,
        nullptr, bias, M, N, K, act, s);
    if (st != TEENY_OK) return st;
  }
  return after_launch("w8a16_linear_forward", s);
}

// linear_backward's MFMA plan: the gradients of a 1x1 convolution over M
// one-pixel images (x [M,1,1,K], w [N,1,1,K], dy [M,1,1,N]); contiguous bf16
// operands with N and K multiples of 8 and 32-bit buffer extents.
static bool linear_bwd_as_conv(int64_t M, int64_t N, int64_t K, teeny_dtype dtype) {
  return dtype == TEENY_BF16 && N % 8 == 0 && K % 8 == 0 && N * K <= 0x7fffffff && M * N * 2 <= 0x7fffff00LL &&
         M * K * 2 <= 0x7fffff00LL;
}

static const teeny_conv2d_params kConv1x1 = {1, 1, 1, 1, 0, 0, 1, TEENY_ACT_NONE};

teeny_status teeny_linear_backward(const void *x, const void *w, const void *dy, void *dx, void *dw, void *db,
                                   int64_t M, int64_t N, int64_t K, int64_t stride_xm, int64_t stride_xk,
                                   int64_t stride_wk, int64_t stride_wn, int64_t stride_dym, int64_t stride_dyn,
                                   int64_t stride_dxm, int64_t stride_dxk, int64_t stride_dwk, int64_t stride_dwn,
                                   int64_t stride_dbn, teeny_dtype dtype, teeny_stream stream) {
  const char *nm = "linear_backward";
  TEENY_REQUIRE(M >= 0 && N >= 0 && K >= 0, TEENY_ERR_SHAPE_MISMATCH, "linear_backward: negative size");
  TEENY_REQUIRE(M <= 0x7fffffff && N <= 0x7fffffff && K <= 0x7fffffff, TEENY_ERR_SHAPE_MISMATCH,
                "linear_backward: size exceeds 2^31-1");
  TEENY_REQUIRE(dtype == TEENY_F32 || dtype == TEENY_BF16, TEENY_ERR_UNSUPPORTED_DTYPE,
                "linear_backward: dtype must be F32 or BF16");
  const bool want_dx = M > 0 && K > 0, want_dw = N > 0 && K > 0, want_db = db != nullptr && N > 0;
  TEENY_REQUIRE((!want_dx || dx != nullptr) && (!want_dw || dw != nullptr), TEENY_ERR_NULL_POINTER,
                "linear_backward: dx/dw");
  TEENY_REQUIRE((!want_dx || N == 0 || (dy != nullptr && w != nullptr)) &&
                    (!want_dw || M == 0 || (dy != nullptr && x != nullptr)) && (!want_db || M == 0 || dy != nullptr),
                TEENY_ERR_NULL_POINTER, "linear_backward: x/w/dy");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool contiguous = stride_xk == 1 && stride_xm == K && stride_wk == 1 && stride_wn == K && stride_dyn == 1 &&
                          stride_dym == N && stride_dxk == 1 && stride_dxm == K && stride_dwk == 1 &&
                          stride_dwn == K;
  const bool conv = contiguous && M > 0 && N > 0 && linear_bwd_as_conv(M, N, K, dtype);
  teeny_status st = TEENY_OK;
  // dx [M, K] = dy [M, N] W [N, K]: C[m, k] = sum_n dy[m, n] w[n, k]
  if (want_dx) {
    if (conv) {
      st = teeny_conv2d_backward_dx(dy, w, dx, M, K, N, 1, 1, 1, 1, &kConv1x1, dtype, TEENY_NHWC, stream);
    } else if (dtype == TEENY_F32) {
      st = launch_generic<float, float, float>(static_cast<const float *>(dy), stride_dym, stride_dyn,
                                               static_cast<const float *>(w), stride_wk, stride_wn,
                                               static_cast<float *>(dx), stride_dxm, stride_dxk, nullptr, nullptr,
                                               nullptr, M, K, N, TEENY_ACT_NONE, s);
    } else {
      st = launch_generic<bf16, bf16, bf16>(static_cast<const bf16 *>(dy), stride_dym, stride_dyn,
                                            static_cast<const bf16 *>(w), stride_wk, stride_wn,
                                            static_cast<bf16 *>(dx), stride_dxm, stride_dxk, nullptr, nullptr,
                                            nullptr, M, K, N, TEENY_ACT_NONE, s);
    }
    if (st != TEENY_OK) return st;
  }
  // dw [N, K] = dy^T x: C[n, k] = sum_m dy[m, n] x[m, k]
  if (want_dw) {
    if (conv) {
      st = teeny_conv2d_backward_dw(dy, x, dw, M, K, N, 1, 1, 1, 1, &kConv1x1, dtype, TEENY_NHWC, stream);
    } else if (dtype == TEENY_F32) {
      st = launch_generic<float, float, float>(static_cast<const float *>(dy), stride_dyn, stride_dym,
                                               static_cast<const float *>(x), stride_xk, stride_xm,
                                               static_cast<float *>(dw), stride_dwn, stride_dwk, nullptr, nullptr,
                                               nullptr, N, K, M, TEENY_ACT_NONE, s);
    } else {
      st = launch_generic<bf16, bf16, bf16>(static_cast<const bf16 *>(dy), stride_dyn, stride_dym,
                                            static_cast<const bf16 *>(x), stride_xk, stride_xm,
                                            static_cast<bf16 *>(dw), stride_dwn, stride_dwk, nullptr, nullptr,
                                            nullptr, N, K, M, TEENY_ACT_NONE, s);
    }
    if (st != TEENY_OK) return st;
  }
  // db [N] = column sums of dy (USE_BIAS)
  if (want_db) {
    const dim3 grid(static_cast<unsigned>(cdiv(N, 64)));
    if (dtype == TEENY_F32)
      hipLaunchKernelGGL(linear_bwd_db<float>, grid, dim3(64), 0, s, static_cast<const float *>(dy), stride_dym,
                         stride_dyn, static_cast<float *>(db), stride_dbn, static_cast<int>(M), static_cast<int>(N));
    else
      hipLaunchKernelGGL(linear_bwd_db<bf16>, grid, dim3(64), 0, s, static_cast<const bf16 *>(dy), stride_dym,
                         stride_dyn, static_cast<bf16 *>(db), stride_dbn, static_cast<int>(M), static_cast<int>(N));
  }
  return after_launch(nm, s);
}

teeny_status teeny_linear_backward_workspace_size(int64_t M, int64_t N, int64_t K, teeny_dtype dtype,
                                                  size_t *bytes) {
  TEENY_REQUIRE(bytes != nullptr, TEENY_ERR_NULL_POINTER, "linear_backward_workspace_size: bytes");
  *bytes = 0;
  TEENY_REQUIRE(M >= 0 && N >= 0 && K >= 0, TEENY_ERR_SHAPE_MISMATCH, "linear_backward_workspace_size: negative size");
  TEENY_REQUIRE(M <= 0x7fffffff && N <= 0x7fffffff && K <= 0x7fffffff, TEENY_ERR_SHAPE_MISMATCH,
                "linear_backward_workspace_size: size exceeds 2^31-1");
  TEENY_REQUIRE(dtype == TEENY_F32 || dtype == TEENY_BF16, TEENY_ERR_UNSUPPORTED_DTYPE,
                "linear_backward_workspace_size: dtype must be F32 or BF16");
  if (M == 0 || N == 0 || K == 0 || !linear_bwd_as_conv(M, N, K, dtype)) return TEENY_OK;
  return teeny_conv2d_backward_workspace_size(M, K, N, 1, 1, 1, 1, &kConv1x1, dtype, TEENY_NHWC, bytes);
}

teeny_status teeny_linear_workspace_size(int64_t M, int64_t N, int64_t K, teeny_dtype dtype,
                                         size_t *bytes) {
  TEENY_REQUIRE(bytes != nullptr, TEENY_ERR_NULL_POINTER, "linear_workspace_size: bytes");
  *bytes = 0;
  TEENY_REQUIRE(M >= 0 && N >= 0 && K >= 0, TEENY_ERR_SHAPE_MISMATCH, "linear_workspace_size: negative size");
  TEENY_REQUIRE(M <= 0x7fffffff && N <= 0x7fffffff && K <= 0x7fffffff, TEENY_ERR_SHAPE_MISMATCH,
                "linear_workspace_size: size exceeds 2^31-1");
  TEENY_REQUIRE(dtype == TEENY_F32 || dtype == TEENY_BF16 || dtype == TEENY_I8, TEENY_ERR_UNSUPPORTED_DTYPE,
                "linear_workspace_size: dtype must be F32, BF16 or I8");
  if (M == 0 || N == 0 || K == 0 || dtype == TEENY_F32) return TEENY_OK;
  if (K % (dtype == TEENY_I8 ? 16 : 8) != 0) return TEENY_OK;  // generic kernel, no scratch
  // contiguous operands, as the MFMA path requires
  const GemmParams p = plain_params(nullptr, K, nullptr, K, nullptr, N, nullptr, nullptr, nullptr, M, N, K);
  *bytes = dtype == TEENY_I8 ? gemm_scratch_bytes<true, kAPlain>(p) : gemm_scratch_bytes<false, kAPlain>(p);
  return TEENY_OK;
}

}  // extern "C"
