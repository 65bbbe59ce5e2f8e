// teeny-quant affine int8/intN quantization on the GPU, bit-exact with
// utilities/teeny-quant/src/quant/affine.rs:47-161 and the group assignment
// of utilities/teeny-quant/src/quant/groups.rs:20-100.
//
// Three kernels, with the reference's two passes:
//   1. quant_minmax: per-group min/max (affine.rs:90-101).  Min and max are
//      exact, so they are reduced with integer atomics on an order-preserving
//      encoding of the fp32 bits; the reduction order cannot change a bit.
//      Each thread scans a contiguous run of elements and issues one atomic
//      pair per group change, so per-channel axis-0 weights cost one atomic
//      pair per run, not per element.
//   2. quant_params: one thread per group applies the reference's scale and
//      zero-point formulas (affine.rs:103-132) in the same fp32 operations.
//   3. quant_values: q = clamp(round(x / scale) as i32 + zp, qmin, qmax)
//      (affine.rs:134-142) with IEEE division (HIP's default correctly
//      rounded fp32 divide), Rust's round-half-away-from-zero and Rust's
//      saturating `as i32` (NaN -> 0).
// The min/max scratch lives in the caller's scales / zero_points arrays,
// which the params kernel then overwrites, so the entry point allocates
// nothing.
#include "common.hpp"

namespace teeny {

constexpr int kQuantMaxDims = 8;
constexpr int kQuantThreads = 256;
constexpr int kQuantRun = 16;  // contiguous elements per thread in the min/max pass

struct QuantShape {
  int64_t shape[kQuantMaxDims];
  int64_t strides[kQuantMaxDims];
  int32_t ndim;
  int32_t gran;
  int32_t axis;
  int32_t pad_;
  int64_t group_size;
  int64_t along;  // ceil(shape[axis] / group_size) for TEENY_GROUP
};

// groups.rs:78-100: PerTensor -> 0; PerChannel -> idx[axis];
// Group -> outer_id * ceil(shape[axis]/group_size) + idx[axis] / group_size,
// where outer_id is the row-major index over the other axes.  With
// s = strides[axis], that index is (i / (s * shape[axis])) * s + i % s.
__host__ __device__ __forceinline__ int64_t group_of(int64_t i, const QuantShape &q) {
  if (q.gran == TEENY_PER_TENSOR) return 0;
  const int64_t s = q.strides[q.axis];
  const int64_t n_axis = q.shape[q.axis];
  const int64_t idx_axis = (i / s) % n_axis;
  if (q.gran == TEENY_PER_CHANNEL) return idx_axis;
  const int64_t outer = (i / (s * n_axis)) * s + (i % s);
  return outer * q.along + idx_axis / q.group_size;
}

// Order-preserving map fp32 -> uint32 (a < b  <=>  key(a) < key(b), with
// -0 < +0).  NaNs never reach it (the reference's `<`/`>` skip them).
__device__ __forceinline__ uint32_t f2key(float f) {
  uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key2f(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}
constexpr uint32_t kMinInit = 0xffffffffu;  // above key(+inf): "no value" (vmin = INFINITY)
constexpr uint32_t kMaxInit = 0x00000000u;  // below key(-inf)

__global__ void quant_init(uint32_t *mins, uint32_t *maxs, int64_t ngroups) {
  int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (g < ngroups) {
    mins[g] = kMinInit;
    maxs[g] = kMaxInit;
  }
}

__global__ __launch_bounds__(kQuantThreads) void quant_minmax(const float *__restrict__ x,
                                                              int64_t n, QuantShape qs,
                                                              uint32_t *mins, uint32_t *maxs,
                                                              uint32_t *groups) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kQuantThreads + threadIdx.x;
  const int64_t begin = t * kQuantRun;
  if (begin >= n) return;
  const int64_t end = begin + kQuantRun < n ? begin + kQuantRun : n;
  int64_t cur = -1;
  uint32_t lo = kMinInit, hi = kMaxInit;
  for (int64_t i = begin; i < end; ++i) {
    const int64_t g = group_of(i, qs);
    if (groups != nullptr) groups[i] = static_cast<uint32_t>(g);
    if (g != cur) {
      if (cur >= 0) {
        if (lo != kMinInit) atomicMin(&mins[cur], lo);
        if (hi != kMaxInit) atomicMax(&maxs[cur], hi);
      }
      cur = g;
      lo = kMinInit;
      hi = kMaxInit;
    }
    const float v = x[i];
    if (v == v) {  // NaN fails both `x < vmin` and `x > vmax` in the reference
      const uint32_t k = f2key(v);
      lo = k < lo ? k : lo;
      hi = k > hi ? k : hi;
    }
  }
  if (lo != kMinInit) atomicMin(&mins[cur], lo);
  if (hi != kMaxInit) atomicMax(&maxs[cur], hi);
}

__device__ __forceinline__ float round_half_away(float v) {
  const float t = truncf(v);
  return fabsf(v - t) >= 0.5f ? t + copysignf(1.0f, v) : t;
}

__device__ __forceinline__ int32_t rust_as_i32(float v) {
  if (v != v) return 0;
  if (v >= 2147483648.0f) return 2147483647;
  if (v <= -2147483648.0f) return static_cast<int32_t>(0x80000000u);
  return static_cast<int32_t>(v);
}

// Reads the min/max keys from (scales, zero_points) and overwrites them with
// the group's params.
__global__ void quant_params(float *scales, int32_t *zero_points, int64_t ngroups, int symmetric,
                             int32_t qmin, int32_t qmax) {
  int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (g >= ngroups) return;
  const uint32_t kmin = reinterpret_cast<uint32_t *>(scales)[g];
  const uint32_t kmax = reinterpret_cast<uint32_t *>(zero_points)[g];
  const float vmin = kmin == kMinInit ? __int_as_float(0x7f800000) : key2f(kmin);
  const float vmax = kmax == kMaxInit ? __int_as_float(0xff800000) : key2f(kmax);
  float lo, hi;
  if (isfinite(vmin)) {
    lo = fminf(vmin, 0.0f);
    hi = fmaxf(vmax, 0.0f);
  } else {
    lo = 0.0f;
    hi = 0.0f;
  }
  if (symmetric) {
    const float amax = fmaxf(fabsf(lo), fabsf(hi));
    scales[g] = amax == 0.0f ? 1.0f : amax / static_cast<float>(qmax);
    zero_points[g] = 0;
  } else {
    const float scale = hi == lo ? 1.0f : (hi - lo) / static_cast<float>(qmax - qmin);
    int32_t zp = rust_as_i32(round_half_away(static_cast<float>(qmin) - lo / scale));
    scales[g] = scale;
    zero_points[g] = zp < qmin ? qmin : (zp > qmax ? qmax : zp);
  }
}

__global__ __launch_bounds__(kQuantThreads) void quant_values(const float *__restrict__ x,
                                                              int64_t n, QuantShape qs,
                                                              const float *__restrict__ scales,
                                                              const int32_t *__restrict__ zps,
                                                              int32_t qmin, int32_t qmax,
                                                              int8_t *__restrict__ q) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kQuantThreads + threadIdx.x;
  if (i >= n) return;
  const int64_t g = group_of(i, qs);
  // i32 add of the reference, widened so the saturated edge stays defined.
  int64_t v = static_cast<int64_t>(rust_as_i32(round_half_away(x[i] / scales[g]))) + zps[g];
  v = v < qmin ? qmin : (v > qmax ? qmax : v);
  q[i] = static_cast<int8_t>(v);
}

__global__ __launch_bounds__(kQuantThreads) void dequant_values(const int8_t *__restrict__ q,
                                                                int64_t n, QuantShape qs,
                                                                const float *__restrict__ scales,
                                                                const int32_t *__restrict__ zps,
                                                                float *__restrict__ out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kQuantThreads + threadIdx.x;
  if (i >= n) return;
  const int64_t g = group_of(i, qs);
  const int32_t zp = zps != nullptr ? zps[g] : 0;
  out[i] = static_cast<float>(static_cast<int32_t>(q[i]) - zp) * scales[g];
}

// Validates the shape/granularity exactly as affine.rs:72-87 and fills qs.
static teeny_status make_shape(const int64_t *shape, int32_t ndim, teeny_granularity gran,
                               int32_t axis, int64_t group_size, QuantShape *qs, int64_t *n,
                               int64_t *ngroups) {
  TEENY_REQUIRE(ndim >= 0 && ndim <= kQuantMaxDims, TEENY_ERR_INVALID_ARGUMENT,
                "quant: ndim must be 0..8");
  TEENY_REQUIRE(ndim == 0 || shape != nullptr, TEENY_ERR_NULL_POINTER, "quant: shape");
  TEENY_REQUIRE(gran >= TEENY_PER_TENSOR && gran <= TEENY_GROUP, TEENY_ERR_INVALID_ARGUMENT,
                "quant: unknown granularity");
  *qs = QuantShape{};
  qs->ndim = ndim;
  qs->gran = gran;
  int64_t total = 1;
  for (int d = 0; d < ndim; ++d) {
    TEENY_REQUIRE(shape[d] >= 0, TEENY_ERR_SHAPE_MISMATCH, "quant: negative dimension");
    qs->shape[d] = shape[d];
    total *= shape[d];
  }
  if (ndim > 0) {
    qs->strides[ndim - 1] = 1;
    for (int d = ndim - 2; d >= 0; --d) qs->strides[d] = qs->strides[d + 1] * shape[d + 1];
  }
  *n = total;
  if (gran == TEENY_PER_TENSOR) {
    *ngroups = 1;
    return TEENY_OK;
  }
  TEENY_REQUIRE(axis >= 0 && axis < ndim, TEENY_ERR_INVALID_AXIS,
                "quant: axis " + std::to_string(axis) + " out of range for rank " +
                    std::to_string(ndim));
  qs->axis = axis;
  if (gran == TEENY_PER_CHANNEL) {
    qs->group_size = 1;
    qs->along = shape[axis];
    *ngroups = shape[axis];
    return TEENY_OK;
  }
  TEENY_REQUIRE(group_size != 0, TEENY_ERR_INVALID_GROUP_SIZE, "quant: group_size is 0");
  TEENY_REQUIRE(group_size > 0, TEENY_ERR_INVALID_GROUP_SIZE, "quant: group_size < 0");
  qs->group_size = group_size;
  qs->along = cdiv(shape[axis], group_size);
  int64_t outer = 1;
  for (int d = 0; d < ndim; ++d)
    if (d != axis) outer *= shape[d];
  *ngroups = outer * qs->along;
  return TEENY_OK;
}

}  // namespace teeny

using namespace teeny;

extern "C" {

teeny_status teeny_quant_num_groups(const int64_t *shape, int32_t ndim,
                                    teeny_granularity granularity, int32_t axis,
                                    int64_t group_size, int64_t *num_groups) {
  TEENY_REQUIRE(num_groups != nullptr, TEENY_ERR_NULL_POINTER, "quant: num_groups");
  QuantShape qs;
  int64_t n = 0;
  return make_shape(shape, ndim, granularity, axis, group_size, &qs, &n, num_groups);
}

teeny_status teeny_quantize_affine(const float *data, const int64_t *shape, int32_t ndim,
                                   teeny_granularity granularity, int32_t axis,
                                   int64_t group_size, int32_t symmetric, int32_t bits,
                                   int8_t *qvalues, float *scales, int32_t *zero_points,
                                   uint32_t *groups, teeny_stream stream) {
  QuantShape qs;
  int64_t n = 0, ngroups = 0;
  teeny_status st = make_shape(shape, ndim, granularity, axis, group_size, &qs, &n, &ngroups);
  if (st != TEENY_OK) return st;
  TEENY_REQUIRE(bits >= 2 && bits <= 8, TEENY_ERR_INVALID_ARGUMENT, "quant: bits must be 2..8");
  TEENY_REQUIRE(scales != nullptr && zero_points != nullptr, TEENY_ERR_NULL_POINTER,
                "quant: scales/zero_points");
  if (n == 0) {
    if (ngroups == 0) return TEENY_OK;
  } else {
    TEENY_REQUIRE(data != nullptr && qvalues != nullptr, TEENY_ERR_NULL_POINTER,
                  "quant: data/qvalues");
  }
  const int32_t qmax = (1 << (bits - 1)) - 1;
  const int32_t qmin = symmetric ? -qmax : -qmax - 1;
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint32_t *mins = reinterpret_cast<uint32_t *>(scales);
  uint32_t *maxs = reinterpret_cast<uint32_t *>(zero_points);
  hipLaunchKernelGGL(quant_init, dim3(cdiv(ngroups, 256)), dim3(256), 0, s, mins, maxs, ngroups);
  if (n > 0) {
    hipLaunchKernelGGL(quant_minmax, dim3(cdiv(cdiv(n, kQuantRun), kQuantThreads)),
                       dim3(kQuantThreads), 0, s, data, n, qs, mins, maxs, groups);
  }
  hipLaunchKernelGGL(quant_params, dim3(cdiv(ngroups, 256)), dim3(256), 0, s, scales, zero_points,
                     ngroups, symmetric, qmin, qmax);
  if (n > 0) {
    hipLaunchKernelGGL(quant_values, dim3(cdiv(n, kQuantThreads)), dim3(kQuantThreads), 0, s,
                       data, n, qs, scales, zero_points, qmin, qmax, qvalues);
  }
  return after_launch("quantize_affine", s);
}

teeny_status teeny_dequantize_affine(const int8_t *qvalues, const float *scales,
                                     const int32_t *zero_points, const int64_t *shape,
                                     int32_t ndim, teeny_granularity granularity, int32_t axis,
                                     int64_t group_size, float *out, teeny_stream stream) {
  QuantShape qs;
  int64_t n = 0, ngroups = 0;
  teeny_status st = make_shape(shape, ndim, granularity, axis, group_size, &qs, &n, &ngroups);
  if (st != TEENY_OK) return st;
  if (n == 0) return TEENY_OK;
  TEENY_REQUIRE(qvalues != nullptr && scales != nullptr && out != nullptr, TEENY_ERR_NULL_POINTER,
                "dequant: qvalues/scales/out");
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(dequant_values, dim3(cdiv(n, kQuantThreads)), dim3(kQuantThreads), 0, s,
                     qvalues, n, qs, scales, zero_points, out);
  return after_launch("dequantize_affine", s);
}

}  // extern "C"
