// Fused chains of unary activations: the reference's PointwiseFuse custom op
// (kernels/teeny-kernels/src/graph/optimizer/ops/pointwise_fuse.rs:73-120),
// which the Anduin pass builds from single-consumer pointwise chains
// (graph/optimizer/anduin.rs:27-60).  Members m_0 .. m_{n-1} are applied in
// order; member i < n-1 leaves its output in scratch_i (the reference keeps
// every intermediate for the backward walk), the last one in y.  Runtime ABI
// (x, y, scratch_0 .. scratch_{n-2}, n_elements), :155-233.
//
// Members and their reference arithmetic (fp32 math; FAST hardware exp and
// reciprocal for bf16 as the single-activation kernels):
//   relu    relu.rs:52-53              max(x, 0)
//   gelu    gelu.rs:53-64              x / (1 + exp(-2c (x + 0.044715 x^3)))
//   silu    sigmoid.rs:144-148         x * (1 / (1 + exp(-x)))
//   sigmoid sigmoid.rs (forward)       1 / (1 + exp(-x))
//   tanh    tanh.rs (forward)          2 * (1 / (1 + exp(-2x))) - 1
// Between members the value is rounded to the tensor's dtype, as the
// reference's members exchange it through dtype-typed scratch buffers: the
// fused chain equals running the members one kernel at a time, bit for bit.
//
// Backward (members with a y-style gradient only: relu, sigmoid, tanh,
// pointwise_fuse.rs:276-279): dx = dy, then for i = n-1 .. 0
// dx = grad_i(dx, y_i), y_i the member's forward output (y for the last,
// scratch_i otherwise), rounded to the dtype after each member:
//   relu dy * (y > 0),  sigmoid dy * (y - y*y),  tanh dy * (1 - y*y).
//
// One pass over HBM: each thread moves one 16-byte vector of every stream,
// so the chain costs 2 + (n-1) tensor passes (x in, y and the kept
// intermediates out) instead of 2n for separate kernels; without scratch
// (inference) it is 2.
#include "common.hpp"

namespace teeny {

constexpr int kPwMax = 8;
constexpr int kPwThreads = 256;

struct PwChain {
  int n;
  int op[kPwMax];
  void *scratch[kPwMax];  // forward outputs of members 0 .. n-2 (entries may be null in forward)
};

template <bool FAST>
__device__ __forceinline__ float pw_apply(int op, float v) {
  switch (op) {
    case TEENY_PW_RELU: return act_relu(v);
    case TEENY_PW_GELU_TANH: return act_gelu<FAST>(v);
    case TEENY_PW_SILU: return act_silu<FAST>(v);
    case TEENY_PW_SIGMOID:
      if constexpr (FAST) return __builtin_amdgcn_rcpf(1.0f + __expf(-v));
      else return 1.0f / (1.0f + expf(-v));
    case TEENY_PW_TANH:
      if constexpr (FAST) return 2.0f * __builtin_amdgcn_rcpf(1.0f + __expf(-2.0f * v)) - 1.0f;
      else return 2.0f * (1.0f / (1.0f + expf(-2.0f * v))) - 1.0f;
    default: return v;
  }
}

__device__ __forceinline__ float pw_grad(int op, float dy, float y) {
  switch (op) {
    case TEENY_PW_RELU: return y > 0.0f ? dy : 0.0f;
    case TEENY_PW_SIGMOID: return dy * (y - y * y);
    case TEENY_PW_TANH: return dy * (1.0f - y * y);
    default: return dy;  // not reached: the host admits y-style members only
  }
}

// Group i of VEC elements: one 16-byte access for the vector kernel (16-byte
// aligned streams), element accesses for the scalar kernel (VEC == 1).
template <typename T, int VEC>
__device__ __forceinline__ void pw_load(const T *p, int64_t i, T (&e)[VEC]) {
  if constexpr (sizeof(T) * VEC == 16) {
    const u32x4 raw = reinterpret_cast<const u32x4 *>(p)[i];
    __builtin_memcpy(e, &raw, 16);
  } else {
#pragma unroll
    for (int k = 0; k < VEC; ++k) e[k] = p[i * VEC + k];
  }
}
template <typename T, int VEC>
__device__ __forceinline__ void pw_store(T *p, int64_t i, const T (&e)[VEC]) {
  if constexpr (sizeof(T) * VEC == 16) {
    u32x4 raw;
    __builtin_memcpy(&raw, e, 16);
    reinterpret_cast<u32x4 *>(p)[i] = raw;
  } else {
#pragma unroll
    for (int k = 0; k < VEC; ++k) p[i * VEC + k] = e[k];
  }
}

// Element group i = VEC consecutive elements starting at begin + VEC i.
template <typename T, int VEC>
__global__ __launch_bounds__(kPwThreads) void pw_forward_kernel(const T *x, T *y,
                                                                PwChain ch, int64_t begin, int64_t groups) {
  constexpr bool fast = !std::is_same<T, float>::value;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kPwThreads + threadIdx.x;
  if (i >= groups) return;
  T e[VEC];
  pw_load<T, VEC>(x + begin, i, e);
  for (int m = 0; m < ch.n; ++m) {
    const int op = ch.op[m];
#pragma unroll
    for (int k = 0; k < VEC; ++k) e[k] = from_f32<T>(pw_apply<fast>(op, to_f32(e[k])));
    if (m + 1 < ch.n) {
      if (ch.scratch[m] != nullptr) pw_store<T, VEC>(static_cast<T *>(ch.scratch[m]) + begin, i, e);
    } else {
      pw_store<T, VEC>(y + begin, i, e);
    }
  }
}

template <typename T, int VEC>
__global__ __launch_bounds__(kPwThreads) void pw_backward_kernel(const T *dy, const T *y, T *dx, PwChain ch, int64_t begin,
                                                                 int64_t groups) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kPwThreads + threadIdx.x;
  if (i >= groups) return;
  T g[VEC], yv[VEC];
  pw_load<T, VEC>(dy + begin, i, g);
  for (int m = ch.n - 1; m >= 0; --m) {
    const T *ym = m + 1 == ch.n ? y : static_cast<const T *>(ch.scratch[m]);
    pw_load<T, VEC>(ym + begin, i, yv);
    const int op = ch.op[m];
#pragma unroll
    for (int k = 0; k < VEC; ++k) g[k] = from_f32<T>(pw_grad(op, to_f32(g[k]), to_f32(yv[k])));
  }
  pw_store<T, VEC>(dx + begin, i, g);
}

static bool pw_aligned(const void *const *ptrs, int n) {
  for (int i = 0; i < n; ++i)
    if (ptrs[i] != nullptr && !aligned(ptrs[i], 16)) return false;
  return true;
}

// Vector kernel over the aligned body, scalar kernel over the tail (or all of
// it when any stream is unaligned).
template <typename T, bool BWD>
static teeny_status pw_launch(const void *a, const void *b, void *out, const PwChain &ch, int64_t n, hipStream_t s,
                              const char *name) {
  constexpr int VEC = 16 / sizeof(T);
  const void *ptrs[3 + kPwMax] = {a, b, out};
  for (int m = 0; m < ch.n; ++m) ptrs[3 + m] = ch.scratch[m];
  int64_t done = 0;
  if (pw_aligned(ptrs, 3 + ch.n)) {
    const int64_t groups = n / VEC;
    if (groups > 0) {
      const int64_t blocks = cdiv(groups, kPwThreads);
      TEENY_REQUIRE(blocks <= 0x7fffffff, TEENY_ERR_SHAPE_MISMATCH, std::string(name) + ": tensor too large");
      if constexpr (BWD)
        hipLaunchKernelGGL((pw_backward_kernel<T, VEC>), dim3(blocks), dim3(kPwThreads), 0, s,
                           static_cast<const T *>(a), static_cast<const T *>(b), static_cast<T *>(out), ch,
                           int64_t{0}, groups);
      else
        hipLaunchKernelGGL((pw_forward_kernel<T, VEC>), dim3(blocks), dim3(kPwThreads), 0, s,
                           static_cast<const T *>(a), static_cast<T *>(out), ch, int64_t{0}, groups);
      done = groups * VEC;
    }
  }
  if (done < n) {
    const int64_t blocks = cdiv(n - done, kPwThreads);
    TEENY_REQUIRE(blocks <= 0x7fffffff, TEENY_ERR_SHAPE_MISMATCH, std::string(name) + ": tensor too large");
    if constexpr (BWD)
      hipLaunchKernelGGL((pw_backward_kernel<T, 1>), dim3(blocks), dim3(kPwThreads), 0, s, static_cast<const T *>(a),
                         static_cast<const T *>(b), static_cast<T *>(out), ch, done, n - done);
    else
      hipLaunchKernelGGL((pw_forward_kernel<T, 1>), dim3(blocks), dim3(kPwThreads), 0, s, static_cast<const T *>(a),
                         static_cast<T *>(out), ch, done, n - done);
  }
  return after_launch(name, s);
}

static teeny_status pw_chain(const int32_t *ops, int32_t n_ops, const void *const *scratch, bool need_scratch,
                             bool bwd, PwChain *ch, const std::string &nm) {
  TEENY_REQUIRE(ops != nullptr, TEENY_ERR_NULL_POINTER, nm + ": ops");
  TEENY_REQUIRE(n_ops >= 1 && n_ops <= kPwMax, TEENY_ERR_INVALID_ARGUMENT,
                nm + ": 1 to " + std::to_string(kPwMax) + " members");
  ch->n = n_ops;
  for (int m = 0; m < kPwMax; ++m) {
    ch->op[m] = 0;
    ch->scratch[m] = nullptr;
  }
  for (int m = 0; m < n_ops; ++m) {
    const int op = ops[m];
    TEENY_REQUIRE(op >= TEENY_PW_RELU && op <= TEENY_PW_TANH, TEENY_ERR_INVALID_ARGUMENT,
                  nm + ": unknown member " + std::to_string(op));
    TEENY_REQUIRE(!bwd || op == TEENY_PW_RELU || op == TEENY_PW_SIGMOID || op == TEENY_PW_TANH,
                  TEENY_ERR_UNSUPPORTED,
                  nm + ": the fused backward takes members with a y-style gradient (relu, sigmoid, tanh)");
    ch->op[m] = op;
    if (m + 1 < n_ops) {
      void *p = scratch != nullptr ? const_cast<void *>(scratch[m]) : nullptr;
      TEENY_REQUIRE(p != nullptr || !need_scratch, TEENY_ERR_NULL_POINTER,
                    nm + ": scratch " + std::to_string(m) + " (member outputs are needed)");
      ch->scratch[m] = p;
    }
  }
  return TEENY_OK;
}

}  // namespace teeny

using namespace teeny;

extern "C" {

teeny_status teeny_pointwise_chain_forward(const void *x, void *y, void *const *scratch, const int32_t *ops,
                                           int32_t n_ops, int64_t n, teeny_dtype dtype, teeny_stream stream) {
  const std::string nm = "pointwise_chain_forward";
  PwChain ch;
  teeny_status st = pw_chain(ops, n_ops, scratch, false, false, &ch, nm);
  if (st != TEENY_OK) return st;
  TEENY_REQUIRE(n >= 0, TEENY_ERR_SHAPE_MISMATCH, nm + ": n_elements < 0");
  TEENY_REQUIRE(dtype == TEENY_F32 || dtype == TEENY_BF16, TEENY_ERR_UNSUPPORTED_DTYPE,
                nm + ": dtype must be F32 or BF16");
  if (n == 0) return TEENY_OK;
  TEENY_REQUIRE(x != nullptr && y != nullptr, TEENY_ERR_NULL_POINTER, nm + ": x/y");
  hipStream_t s = static_cast<hipStream_t>(stream);
  return dtype == TEENY_F32 ? pw_launch<float, false>(x, nullptr, y, ch, n, s, nm.c_str())
                            : pw_launch<bf16, false>(x, nullptr, y, ch, n, s, nm.c_str());
}

teeny_status teeny_pointwise_chain_backward(const void *dy, const void *y, void *dx, const void *const *scratch,
                                            const int32_t *ops, int32_t n_ops, int64_t n, teeny_dtype dtype,
                                            teeny_stream stream) {
  const std::string nm = "pointwise_chain_backward";
  PwChain ch;
  teeny_status st = pw_chain(ops, n_ops, scratch, true, true, &ch, nm);
  if (st != TEENY_OK) return st;
  TEENY_REQUIRE(n >= 0, TEENY_ERR_SHAPE_MISMATCH, nm + ": n_elements < 0");
  TEENY_REQUIRE(dtype == TEENY_F32 || dtype == TEENY_BF16, TEENY_ERR_UNSUPPORTED_DTYPE,
                nm + ": dtype must be F32 or BF16");
  if (n == 0) return TEENY_OK;
  TEENY_REQUIRE(dy != nullptr && y != nullptr && dx != nullptr, TEENY_ERR_NULL_POINTER, nm + ": dy/y/dx");
  hipStream_t s = static_cast<hipStream_t>(stream);
  return dtype == TEENY_F32 ? pw_launch<float, true>(dy, y, dx, ch, n, s, nm.c_str())
                            : pw_launch<bf16, true>(dy, y, dx, ch, n, s, nm.c_str());
}

}  // extern "C"
