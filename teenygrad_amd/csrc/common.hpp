// Shared host/device helpers for the teeny_hip library (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "../../include/teeny_hip.h"

namespace teeny {

// ── host-side error plumbing ────────────────────────────────────────────────
void set_error(const std::string &msg);
teeny_status fail(teeny_status code, const std::string &msg);
teeny_status hip_fail(hipError_t err, const char *what);
// Called after every kernel launch: checks the launch and honours TEENY_HIP_SYNC.
teeny_status after_launch(const char *what, hipStream_t stream);
// Compute units of the current device (cached per device ordinal).
int device_cu_count();
// Caller-owned device scratch attached to a stream with
// teeny_hip_stream_set_workspace ({nullptr, 0} if none).  Operators never
// allocate: paths that need scratch (split-K partial sums, the
// space-to-depth copy of a stride-2 conv) run only when it is large enough.
struct Scratch {
  void *ptr = nullptr;
  size_t bytes = 0;
};
Scratch stream_scratch(hipStream_t stream);

#define TEENY_CHECK_HIP(expr)                                                      \
  do {                                                                             \
    hipError_t e_ = (expr);                                                        \
    if (e_ != hipSuccess) return ::teeny::hip_fail(e_, #expr);                     \
  } while (0)

#define TEENY_REQUIRE(cond, code, msg)                                             \
  do {                                                                             \
    if (!(cond)) return ::teeny::fail((code), (msg));                              \
  } while (0)

inline bool aligned(const void *p, size_t a) {
  return (reinterpret_cast<uintptr_t>(p) % a) == 0;
}

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ── device-side types ───────────────────────────────────────────────────────
typedef __bf16 bf16;
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(bf16 v) { return static_cast<float>(v); }
template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
// Round-to-nearest-even (hardware v_cvt_pk_bf16_f32 on gfx950).
template <> __device__ __forceinline__ bf16 from_f32<bf16>(float v) { return static_cast<bf16>(v); }

// ── activations (fp32 math) ─────────────────────────────────────────────────
// relu: nn/activation/relu.rs:27-64 (maximum(x, 0)); NaN propagates.
// gelu: nn/activation/gelu.rs:58-64, y = x / (1 + exp(-2c (x + 0.044715 x^3))).
// silu: nn/activation/sigmoid.rs:146-148, y = x * (1 / (1 + exp(-x))).
//
// FAST selects the hardware transcendental path (v_exp_f32 on x*log2(e), and
// v_rcp_f32 instead of an IEEE divide).  Its relative error is a few 1e-7
// plus |arg| * 6e-8 from rounding the exp2 argument: far below bf16's
// 3.9e-3 ulp, so bf16 kernels use it; fp32 kernels use the correctly rounded
// divide and the full-accuracy expf so that fp32 parity holds to 1e-5.
// At [16384, 4096] bf16 the accurate path would cost about as much VALU time
// as the HBM traffic itself, which is why the split exists.
__device__ __forceinline__ float act_relu(float x) { return x < 0.0f ? 0.0f : x; }
template <bool FAST> __device__ __forceinline__ float act_gelu(float x) {
  const float neg2c = -1.5957691216057308f;  // -2 * sqrt(2/pi)
  const float coeff = 0.044715f;
  if constexpr (FAST) {
    // exp(-2c (x + a x^3)) = exp2(x (k1 + k3 x^2)) with the constants folded:
    // k1 = -2c log2(e), k3 = a k1 (one v_exp_f32, no separate cube or scaling)
    const float k1 = -2.302208198144325f, k3 = -0.1029432395800235f;
    return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * __builtin_fmaf(k3, x * x, k1)));
  } else {
    float inner = x + coeff * x * x * x;
    return x / (1.0f + expf(neg2c * inner));
  }
}
template <bool FAST> __device__ __forceinline__ float act_silu(float x) {
  if constexpr (FAST) {
    return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x));
  } else {
    float s = 1.0f / (1.0f + expf(-x));
    return x * s;
  }
}
// Runtime-selected activation (workgroup-uniform `act`), for epilogues where
// one kernel serves every activation.
__device__ __forceinline__ float apply_act_rt(float x, int act) {
  switch (act) {
    case TEENY_ACT_RELU: return act_relu(x);
    case TEENY_ACT_GELU_TANH: return act_gelu<true>(x);
    case TEENY_ACT_SILU: return act_silu<true>(x);
    default: return x;
  }
}
template <int ACT, bool FAST> __device__ __forceinline__ float apply_act(float x) {
  if constexpr (ACT == TEENY_ACT_RELU) return act_relu(x);
  else if constexpr (ACT == TEENY_ACT_GELU_TANH) return act_gelu<FAST>(x);
  else if constexpr (ACT == TEENY_ACT_SILU) return act_silu<FAST>(x);
  else return x;
}

// ── launch geometry ─────────────────────────────────────────────────────────
// Workgroup id -> logical tile id such that each of the 8 XCDs (which receive
// workgroups round-robin, each with its own L2) gets one contiguous run of
// tile ids; neighbouring tiles that share operands then share an L2.
__device__ __forceinline__ int xcd_remap(int bid, int nwg) {
  const int q = nwg >> 3, r = nwg & 7;
  const int xcd = bid & 7, slot = bid >> 3;
  return xcd < r ? xcd * (q + 1) + slot : r * (q + 1) + (xcd - r) * q + slot;
}

// ── wavefront reductions (wave64) ───────────────────────────────────────────
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}
// The same total through DPP, with no LDS round trips (all 64 lanes must be
// active): pair and quad sums (quad_perm), 8- and 16-lane sums (row half
// mirror, row mirror), then the row broadcasts that leave the total in lane
// 63, read back as a wave-uniform value.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_add(float v) {
  return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xf, false));
}
__device__ __forceinline__ float wave_total(float v) {
  v = dpp_add<0xb1, 0xf>(v);   // quad_perm [1, 0, 3, 2]
  v = dpp_add<0x4e, 0xf>(v);   // quad_perm [2, 3, 0, 1]
  v = dpp_add<0x141, 0xf>(v);  // row_half_mirror
  v = dpp_add<0x140, 0xf>(v);  // row_mirror
  v = dpp_add<0x142, 0xa>(v);  // row_bcast:15 into rows 1 and 3
  v = dpp_add<0x143, 0xc>(v);  // row_bcast:31 into rows 2 and 3
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

}  // namespace teeny
