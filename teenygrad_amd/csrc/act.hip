// Elementwise activations: relu / gelu-tanh / silu, fp32 and bf16.
//
// Reference kernels (one BLOCK_SIZE-element tile per program id, masked tail):
//   relu_forward  kernels/teeny-kernels/src/nn/activation/relu.rs:27-64
//   gelu_forward  kernels/teeny-kernels/src/nn/activation/gelu.rs:31-78
//   silu_forward  kernels/teeny-kernels/src/nn/activation/sigmoid.rs:119-158
// and their gradients (dy and the saved tensor in, dx out):
//   relu_backward kernels/teeny-kernels/src/nn/activation/relu.rs:67-117
//   gelu_backward kernels/teeny-kernels/src/nn/activation/gelu.rs:81-139
//   silu_backward kernels/teeny-kernels/src/nn/activation/sigmoid.rs:161-210
//
// MI355X design: the op moves 2 bytes in and 2 out per bf16 element with a
// handful of VALU ops, so it is bound by HBM.  Each thread moves one 16-byte
// vector; lanes of a wave touch consecutive 16-byte chunks so every load
// instruction is one fully coalesced 1 KiB request; both the loads and the
// stores are non-temporal (the data streams through once).  With ~16 VGPRs
// the kernel runs at 8 waves per SIMD; a [16384, 4096] bf16 tensor is 16384
// workgroups of 512 threads (256-thread workgroups: the forward the same,
// the three gradients 64.0-65.8 against 63.2-64.4 us; 1024 threads: the
// forward 42.5 -> 44.5 us).  Measured on MI355X at the settled clock over rotating 128 MiB
// buffers (GELU, [16384, 4096] bf16): one vector per thread with
// non-temporal loads 42.3 us (0.79 of 8 TB/s), against 45.1 us for two
// vectors with temporal loads, 43.4-43.5 us for either change alone, 46.5 us
// for four vectors and 46-47 us for persistent grid-stride loops; a device
// copy (hipMemcpyAsync) takes 50.9 us.  Unaligned pointers or a ragged tail
// take a scalar kernel.  The backward kernels have the same shape with two
// input streams, 6 bytes per bf16 element (GELU gradient 69.9 -> 62.5 us,
// 0.81 of 8 TB/s).
#include "common.hpp"

namespace teeny {

constexpr int kActThreads = 512;
constexpr int kActUnroll = 1;

template <typename T, int ACT>
__device__ __forceinline__ T act_one(T v) {
  constexpr bool fast = !std::is_same<T, float>::value;
  return from_f32<T>(apply_act<ACT, fast>(to_f32(v)));
}

// x and y may alias: every element is read and written by the same thread.
template <typename T, int ACT>
__global__ __launch_bounds__(kActThreads) void act_vec_kernel(const T *x, T *y, int64_t n_vec) {
  constexpr int VEC = 16 / sizeof(T);
  typedef u32x4 raw_t;
  const int64_t base = static_cast<int64_t>(blockIdx.x) * (kActThreads * kActUnroll) + threadIdx.x;
  raw_t r[kActUnroll];
#pragma unroll
  for (int u = 0; u < kActUnroll; ++u) {
    int64_t v = base + u * kActThreads;
    if (v < n_vec) r[u] = __builtin_nontemporal_load(reinterpret_cast<const raw_t *>(x) + v);
  }
#pragma unroll
  for (int u = 0; u < kActUnroll; ++u) {
    int64_t v = base + u * kActThreads;
    if (v < n_vec) {
      T e[VEC];
      __builtin_memcpy(e, &r[u], 16);
#pragma unroll
      for (int i = 0; i < VEC; ++i) e[i] = act_one<T, ACT>(e[i]);
      __builtin_memcpy(&r[u], e, 16);
      __builtin_nontemporal_store(r[u], reinterpret_cast<raw_t *>(y) + v);
    }
  }
}

template <typename T, int ACT>
__global__ __launch_bounds__(kActThreads) void act_scalar_kernel(const T *x, T *y, int64_t begin,
                                                                 int64_t n) {
  int64_t i = begin + static_cast<int64_t>(blockIdx.x) * kActThreads + threadIdx.x;
  if (i < n) y[i] = act_one<T, ACT>(x[i]);
}

template <typename T, int ACT>
static teeny_status launch_act(const void *xv, void *yv, int64_t n, hipStream_t s,
                               const char *name) {
  const T *x = static_cast<const T *>(xv);
  T *y = static_cast<T *>(yv);
  constexpr int VEC = 16 / sizeof(T);
  int64_t done = 0;
  if (aligned(x, 16) && aligned(y, 16)) {
    int64_t n_vec = n / VEC;
    if (n_vec > 0) {
      int64_t blocks = cdiv(n_vec, kActThreads * kActUnroll);
      TEENY_REQUIRE(blocks <= 0x7fffffff, TEENY_ERR_SHAPE_MISMATCH, "tensor too large");
      hipLaunchKernelGGL((act_vec_kernel<T, ACT>), dim3(blocks), dim3(kActThreads), 0, s, x, y,
                         n_vec);
      teeny_status st = after_launch(name, s);
      if (st != TEENY_OK) return st;
    }
    done = n_vec * VEC;
  }
  if (done < n) {
    int64_t blocks = cdiv(n - done, kActThreads);
    TEENY_REQUIRE(blocks <= 0x7fffffff, TEENY_ERR_SHAPE_MISMATCH, "tensor too large");
    hipLaunchKernelGGL((act_scalar_kernel<T, ACT>), dim3(blocks), dim3(kActThreads), 0, s, x, y,
                       done, n);
    return after_launch(name, s);
  }
  return TEENY_OK;
}

template <int ACT>
static teeny_status act_entry(const void *x, void *y, int64_t n, teeny_dtype dtype,
                              teeny_stream stream, const char *name) {
  TEENY_REQUIRE(n >= 0, TEENY_ERR_SHAPE_MISMATCH, std::string(name) + ": n_elements < 0");
  if (n == 0) return TEENY_OK;
  TEENY_REQUIRE(x != nullptr && y != nullptr, TEENY_ERR_NULL_POINTER, std::string(name) + ": x/y");
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case TEENY_F32: return launch_act<float, ACT>(x, y, n, s, name);
    case TEENY_BF16: return launch_act<bf16, ACT>(x, y, n, s, name);
    default:
      return fail(TEENY_ERR_UNSUPPORTED_DTYPE, std::string(name) + ": dtype must be F32 or BF16");
  }
}

// ── backward ────────────────────────────────────────────────────────────────
// Gradient of each activation, in the reference's arithmetic:
//   relu (relu.rs:105-107): dx = y > 0 ? dy : 0, with y the forward output
//     (a NaN y gives 0, as the reference's where_ does).
//   gelu (gelu.rs:125-130): inner = x + a x^3, s = 1/(1 + exp(-2c inner)),
//     t = 2s - 1 (= tanh(c inner)), dx = dy (0.5 (1 + t) + x 0.5 (1 - t^2) c (1 + 3a x^2)).
//   silu (sigmoid.rs:198-201): s = 1/(1 + exp(-x)), y = x s, dx = dy (s + y - y s).
// FAST as for the forward activations: bf16 kernels use the hardware exp and
// reciprocal, fp32 kernels the full-accuracy expf and IEEE divide.
template <int ACT, bool FAST>
__device__ __forceinline__ float act_grad(float dy, float v) {
  if constexpr (ACT == TEENY_ACT_RELU) {
    return v > 0.0f ? dy : 0.0f;
  } else if constexpr (ACT == TEENY_ACT_GELU_TANH) {
    const float c = 0.7978845608028654f;      // sqrt(2/pi)
    const float neg2c = -1.5957691216057308f;  // -2 * sqrt(2/pi)
    const float a = 0.044715f;
    const float inner = v + a * v * v * v;
    const float e = FAST ? __expf(neg2c * inner) : expf(neg2c * inner);
    const float s = FAST ? __builtin_amdgcn_rcpf(1.0f + e) : 1.0f / (1.0f + e);
    const float t = 2.0f * s - 1.0f;
    const float sech2 = 1.0f - t * t;
    const float dinner = c * (1.0f + 3.0f * a * v * v);
    return dy * (0.5f * (1.0f + t) + v * 0.5f * sech2 * dinner);
  } else {
    const float e = FAST ? __expf(-v) : expf(-v);
    const float s = FAST ? __builtin_amdgcn_rcpf(1.0f + e) : 1.0f / (1.0f + e);
    const float y = v * s;
    return dy * (s + y - y * s);
  }
}

template <typename T, int ACT>
__device__ __forceinline__ T grad_one(T dy, T v) {
  constexpr bool fast = !std::is_same<T, float>::value;
  return from_f32<T>(act_grad<ACT, fast>(to_f32(dy), to_f32(v)));
}

// dx may alias dy or v: every element is read and written by the same thread.
template <typename T, int ACT>
__global__ __launch_bounds__(kActThreads) void act_bwd_vec_kernel(const T *dy, const T *v, T *dx,
                                                                  int64_t n_vec) {
  constexpr int VEC = 16 / sizeof(T);
  const int64_t base = static_cast<int64_t>(blockIdx.x) * (kActThreads * kActUnroll) + threadIdx.x;
  u32x4 rd[kActUnroll], rv[kActUnroll];
#pragma unroll
  for (int u = 0; u < kActUnroll; ++u) {
    const int64_t i = base + u * kActThreads;
    if (i < n_vec) {
      rd[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(dy) + i);
      rv[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(v) + i);
    }
  }
#pragma unroll
  for (int u = 0; u < kActUnroll; ++u) {
    const int64_t i = base + u * kActThreads;
    if (i < n_vec) {
      T d[VEC], e[VEC];
      __builtin_memcpy(d, &rd[u], 16);
      __builtin_memcpy(e, &rv[u], 16);
#pragma unroll
      for (int k = 0; k < VEC; ++k) d[k] = grad_one<T, ACT>(d[k], e[k]);
      u32x4 r;
      __builtin_memcpy(&r, d, 16);
      __builtin_nontemporal_store(r, reinterpret_cast<u32x4 *>(dx) + i);
    }
  }
}

template <typename T, int ACT>
__global__ __launch_bounds__(kActThreads) void act_bwd_scalar_kernel(const T *dy, const T *v, T *dx,
                                                                     int64_t begin, int64_t n) {
  const int64_t i = begin + static_cast<int64_t>(blockIdx.x) * kActThreads + threadIdx.x;
  if (i < n) dx[i] = grad_one<T, ACT>(dy[i], v[i]);
}

template <typename T, int ACT>
static teeny_status launch_act_bwd(const void *dyv, const void *vv, void *dxv, int64_t n,
                                   hipStream_t s, const char *name) {
  const T *dy = static_cast<const T *>(dyv);
  const T *v = static_cast<const T *>(vv);
  T *dx = static_cast<T *>(dxv);
  constexpr int VEC = 16 / sizeof(T);
  int64_t done = 0;
  if (aligned(dy, 16) && aligned(v, 16) && aligned(dx, 16)) {
    const int64_t n_vec = n / VEC;
    if (n_vec > 0) {
      const int64_t blocks = cdiv(n_vec, kActThreads * kActUnroll);
      TEENY_REQUIRE(blocks <= 0x7fffffff, TEENY_ERR_SHAPE_MISMATCH, "tensor too large");
      hipLaunchKernelGGL((act_bwd_vec_kernel<T, ACT>), dim3(blocks), dim3(kActThreads), 0, s, dy,
                         v, dx, n_vec);
      teeny_status st = after_launch(name, s);
      if (st != TEENY_OK) return st;
    }
    done = n_vec * VEC;
  }
  if (done < n) {
    const int64_t blocks = cdiv(n - done, kActThreads);
    TEENY_REQUIRE(blocks <= 0x7fffffff, TEENY_ERR_SHAPE_MISMATCH, "tensor too large");
    hipLaunchKernelGGL((act_bwd_scalar_kernel<T, ACT>), dim3(blocks), dim3(kActThreads), 0, s, dy,
                       v, dx, done, n);
    return after_launch(name, s);
  }
  return TEENY_OK;
}

template <int ACT>
static teeny_status act_bwd_entry(const void *dy, const void *v, void *dx, int64_t n,
                                  teeny_dtype dtype, teeny_stream stream, const char *name) {
  TEENY_REQUIRE(n >= 0, TEENY_ERR_SHAPE_MISMATCH, std::string(name) + ": n_elements < 0");
  if (n == 0) return TEENY_OK;
  TEENY_REQUIRE(dy != nullptr && v != nullptr && dx != nullptr, TEENY_ERR_NULL_POINTER,
                std::string(name) + ": dy/saved/dx");
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case TEENY_F32: return launch_act_bwd<float, ACT>(dy, v, dx, n, s, name);
    case TEENY_BF16: return launch_act_bwd<bf16, ACT>(dy, v, dx, n, s, name);
    default:
      return fail(TEENY_ERR_UNSUPPORTED_DTYPE, std::string(name) + ": dtype must be F32 or BF16");
  }
}

}  // namespace teeny

using namespace teeny;

extern "C" {

teeny_status teeny_relu_forward(const void *x, void *y, int64_t n_elements, teeny_dtype dtype,
                                teeny_stream stream) {
  return act_entry<TEENY_ACT_RELU>(x, y, n_elements, dtype, stream, "relu_forward");
}

teeny_status teeny_gelu_forward(const void *x, void *y, int64_t n_elements, teeny_dtype dtype,
                                teeny_stream stream) {
  return act_entry<TEENY_ACT_GELU_TANH>(x, y, n_elements, dtype, stream, "gelu_forward");
}

teeny_status teeny_silu_forward(const void *x, void *y, int64_t n_elements, teeny_dtype dtype,
                                teeny_stream stream) {
  return act_entry<TEENY_ACT_SILU>(x, y, n_elements, dtype, stream, "silu_forward");
}

teeny_status teeny_relu_backward(const void *dy, const void *y, void *dx, int64_t n_elements,
                                 teeny_dtype dtype, teeny_stream stream) {
  return act_bwd_entry<TEENY_ACT_RELU>(dy, y, dx, n_elements, dtype, stream, "relu_backward");
}

teeny_status teeny_gelu_backward(const void *dy, const void *x, void *dx, int64_t n_elements,
                                 teeny_dtype dtype, teeny_stream stream) {
  return act_bwd_entry<TEENY_ACT_GELU_TANH>(dy, x, dx, n_elements, dtype, stream, "gelu_backward");
}

teeny_status teeny_silu_backward(const void *dy, const void *x, void *dx, int64_t n_elements,
                                 teeny_dtype dtype, teeny_stream stream) {
  return act_bwd_entry<TEENY_ACT_SILU>(dy, x, dx, n_elements, dtype, stream, "silu_backward");
}

}  // extern "C"
