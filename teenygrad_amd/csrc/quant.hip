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
//
// Contiguous groups (per-tensor, and per-channel over axis 0: group g is the
// elements [g L, (g + 1) L) with L = n / shape[0]), the layout of every
// weight teeny-quant quantizes per output channel, take faster forms of
// passes 1 and 3: a workgroup reduces one segment of <= 16384 elements of
// one group with 16-byte loads, wave shuffles and one LDS exchange, then
// issues a single atomic pair; the values pass maps four elements per thread
// (one 16-byte load, one 4-byte store) with one 32-bit division for the
// group of the first.  Group ids are written only when asked for.
#include <algorithm>

#include "common.hpp"

namespace teeny {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

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

// ── contiguous groups ──
constexpr int64_t kSegMax = 16384;  // elements per workgroup in the min/max pass

__device__ __forceinline__ void seg_fold(float v, uint32_t &lo, uint32_t &hi) {
  if (v == v) {  // NaN fails both `x < vmin` and `x > vmax` in the reference
    const uint32_t k = f2key(v);
    lo = k < lo ? k : lo;
    hi = k > hi ? k : hi;
  }
}

// Workgroup s reduces elements [g L + j seg, min(g L + (j + 1) seg, (g + 1) L))
// of group g = s / segs (j = s % segs) and folds them into the group's keys.
__global__ __launch_bounds__(kQuantThreads) void quant_minmax_seg(const float *__restrict__ x, int64_t L,
                                                                  int64_t seg, int64_t segs, uint32_t *mins,
                                                                  uint32_t *maxs) {
  __shared__ uint32_t red[2][kQuantThreads / 64];
  const int64_t g = blockIdx.x / segs;
  const int64_t begin = g * L + (blockIdx.x % segs) * seg;
  const int64_t end = begin + seg < (g + 1) * L ? begin + seg : (g + 1) * L;
  const int tid = threadIdx.x;
  uint32_t lo = kMinInit, hi = kMaxInit;
  // scalar head up to a 16-byte boundary, 16-byte body, scalar tail
  const int64_t up = (begin + 3) & ~static_cast<int64_t>(3);
  const int64_t head = up < end ? up : end;
  if (begin + tid < head) seg_fold(x[begin + tid], lo, hi);
  const int64_t body_end = head + ((end - head) & ~static_cast<int64_t>(3));
  for (int64_t i = head + 4 * tid; i < body_end; i += 4 * kQuantThreads) {
    const f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(x + i));
    seg_fold(v[0], lo, hi);
    seg_fold(v[1], lo, hi);
    seg_fold(v[2], lo, hi);
    seg_fold(v[3], lo, hi);
  }
  if (body_end + tid < end) seg_fold(x[body_end + tid], lo, hi);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const uint32_t l2 = __shfl_xor(lo, off, 64), h2 = __shfl_xor(hi, off, 64);
    lo = l2 < lo ? l2 : lo;
    hi = h2 > hi ? h2 : hi;
  }
  if ((tid & 63) == 0) {
    red[0][tid >> 6] = lo;
    red[1][tid >> 6] = hi;
  }
  __syncthreads();
  if (tid == 0) {
#pragma unroll
    for (int w = 1; w < kQuantThreads / 64; ++w) {
      lo = red[0][w] < lo ? red[0][w] : lo;
      hi = red[1][w] > hi ? red[1][w] : hi;
    }
    if (lo != kMinInit) atomicMin(&mins[g], lo);
    if (hi != kMaxInit) atomicMax(&maxs[g], hi);
  }
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

// A group's scale and zero point from its min/max keys (affine.rs:103-132).
__device__ __forceinline__ void group_params(uint32_t kmin, uint32_t kmax, int symmetric, int32_t qmin, int32_t qmax,
                                             float &scale_out, int32_t &zp_out) {
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
    scale_out = amax == 0.0f ? 1.0f : amax / static_cast<float>(qmax);
    zp_out = 0;
  } else {
    const float scale = hi == lo ? 1.0f : (hi - lo) / static_cast<float>(qmax - qmin);
    int32_t zp = rust_as_i32(round_half_away(static_cast<float>(qmin) - lo / scale));
    scale_out = scale;
    zp_out = zp < qmin ? qmin : (zp > qmax ? qmax : zp);
  }
}

// Reads the min/max keys from (scales, zero_points) and overwrites them with
// the group's params.
__global__ void quant_params(float *scales, int32_t *zero_points, int64_t ngroups, int symmetric,
                             int32_t qmin, int32_t qmax) {
  int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (g >= ngroups) return;
  float sc;
  int32_t zp;
  group_params(reinterpret_cast<uint32_t *>(scales)[g], reinterpret_cast<uint32_t *>(zero_points)[g], symmetric,
               qmin, qmax, sc, zp);
  scales[g] = sc;
  zero_points[g] = zp;
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

// The values pass over contiguous groups of L >= 4 elements, n < 2^31 and
// 16-byte aligned x: four elements per thread (at most one group boundary
// among them).
__device__ __forceinline__ int8_t quant_one(float x, float scale, int32_t zp, int32_t qmin, int32_t qmax) {
  int64_t v = static_cast<int64_t>(rust_as_i32(round_half_away(x / scale))) + zp;
  v = v < qmin ? qmin : (v > qmax ? qmax : v);
  return static_cast<int8_t>(v);
}

// Both passes in one kernel for contiguous groups of L <= 1024 VPT elements
// with L % 4 == 0 (per-channel axis-0 weights): a workgroup holds its group
// in registers (VPT 16-byte vectors per thread), reduces min/max, derives the
// scale and zero point, and quantizes from the registers, so x is read once.
template <int VPT>
__global__ __launch_bounds__(kQuantThreads) void quant_rows_fused(const float *__restrict__ x, int L, int symmetric,
                                                                  int32_t qmin, int32_t qmax, int8_t *__restrict__ q,
                                                                  float *__restrict__ scales,
                                                                  int32_t *__restrict__ zps,
                                                                  uint32_t *__restrict__ groups) {
  __shared__ uint32_t red[2][kQuantThreads / 64];
  __shared__ float s_scale;
  __shared__ int32_t s_zp;
  const int tid = threadIdx.x;
  const int64_t g = blockIdx.x;
  const float *row = x + g * L;
  f32x4 v[VPT];
  uint32_t lo = kMinInit, hi = kMaxInit;
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int c = 4 * (tid + kQuantThreads * j);
    if (c < L) {
      v[j] = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(row + c));
      seg_fold(v[j][0], lo, hi);
      seg_fold(v[j][1], lo, hi);
      seg_fold(v[j][2], lo, hi);
      seg_fold(v[j][3], lo, hi);
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const uint32_t l2 = __shfl_xor(lo, off, 64), h2 = __shfl_xor(hi, off, 64);
    lo = l2 < lo ? l2 : lo;
    hi = h2 > hi ? h2 : hi;
  }
  if ((tid & 63) == 0) {
    red[0][tid >> 6] = lo;
    red[1][tid >> 6] = hi;
  }
  __syncthreads();
  if (tid == 0) {
#pragma unroll
    for (int w = 1; w < kQuantThreads / 64; ++w) {
      lo = red[0][w] < lo ? red[0][w] : lo;
      hi = red[1][w] > hi ? red[1][w] : hi;
    }
    float sc;
    int32_t zp;
    group_params(lo, hi, symmetric, qmin, qmax, sc, zp);
    s_scale = sc;
    s_zp = zp;
    scales[g] = sc;
    zps[g] = zp;
  }
  __syncthreads();
  const float sc = s_scale;
  const int32_t zp = s_zp;
  int8_t *qrow = q + g * L;
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int c = 4 * (tid + kQuantThreads * j);
    if (c < L) {
      uint32_t packed = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        packed |= static_cast<uint32_t>(static_cast<uint8_t>(quant_one(v[j][e], sc, zp, qmin, qmax))) << (8 * e);
      *reinterpret_cast<uint32_t *>(qrow + c) = packed;
      if (groups != nullptr) {
        const uint32_t gg = static_cast<uint32_t>(g);
        *reinterpret_cast<u32x4 *>(groups + g * L + c) = u32x4{gg, gg, gg, gg};
      }
    }
  }
}

__global__ __launch_bounds__(kQuantThreads) void quant_values_seg(const float *__restrict__ x, int n, int L,
                                                                  const float *__restrict__ scales,
                                                                  const int32_t *__restrict__ zps, int32_t qmin,
                                                                  int32_t qmax, int8_t *__restrict__ q,
                                                                  uint32_t *__restrict__ groups) {
  const int i = (blockIdx.x * kQuantThreads + threadIdx.x) * 4;
  if (i >= n) return;
  const uint32_t g0 = static_cast<uint32_t>(i) / static_cast<uint32_t>(L);
  const int r = i - static_cast<int>(g0) * L;
  const float s0 = scales[g0];
  const int32_t z0 = zps[g0];
  if (i + 4 <= n) {
    const f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(x + i));
    const bool cross = r + 4 > L;  // elements L - r .. 3 belong to group g0 + 1
    const float s1 = cross ? scales[g0 + 1] : s0;
    const int32_t z1 = cross ? zps[g0 + 1] : z0;
    uint32_t packed = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const bool next = r + e >= L;
      const int8_t b = quant_one(v[e], next ? s1 : s0, next ? z1 : z0, qmin, qmax);
      packed |= static_cast<uint32_t>(static_cast<uint8_t>(b)) << (8 * e);
      if (groups != nullptr) groups[i + e] = next ? g0 + 1 : g0;
    }
    *reinterpret_cast<uint32_t *>(q + i) = packed;
    return;
  }
  for (int e = 0; i + e < n; ++e) {  // the last, partial quad
    const bool next = r + e >= L;
    q[i + e] = quant_one(x[i + e], next ? scales[g0 + 1] : s0, next ? zps[g0 + 1] : z0, qmin, qmax);
    if (groups != nullptr) groups[i + e] = next ? g0 + 1 : g0;
  }
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
  // contiguous groups of equal length L: per-tensor, or per-channel over the
  // leading axis (group g = elements [g L, (g + 1) L))
  const bool contiguous = granularity == TEENY_PER_TENSOR || (granularity == TEENY_PER_CHANNEL && axis == 0);
  const int64_t L = ngroups > 0 ? n / ngroups : 0;
  const bool seg = n > 0 && contiguous && L >= 4 && n <= 0x7fffffff && aligned(data, 16) && aligned(qvalues, 4);
  // per-channel axis 0 with rows of <= 16384 elements, a multiple of 4: one kernel
  const bool fused = seg && granularity == TEENY_PER_CHANNEL && L % 4 == 0 && L <= 4 * kQuantThreads * 16 &&
                     (groups == nullptr || aligned(groups, 16));
  if (fused) {
    const dim3 grid(static_cast<unsigned>(ngroups));
    const int Li = static_cast<int>(L);
    if (L <= 4 * kQuantThreads * 4)
      hipLaunchKernelGGL(quant_rows_fused<4>, grid, dim3(kQuantThreads), 0, s, data, Li, symmetric, qmin, qmax,
                         qvalues, scales, zero_points, groups);
    else if (L <= 4 * kQuantThreads * 8)
      hipLaunchKernelGGL(quant_rows_fused<8>, grid, dim3(kQuantThreads), 0, s, data, Li, symmetric, qmin, qmax,
                         qvalues, scales, zero_points, groups);
    else
      hipLaunchKernelGGL(quant_rows_fused<16>, grid, dim3(kQuantThreads), 0, s, data, Li, symmetric, qmin, qmax,
                         qvalues, scales, zero_points, groups);
    return after_launch("quantize_affine", s);
  }
  hipLaunchKernelGGL(quant_init, dim3(cdiv(ngroups, 256)), dim3(256), 0, s, mins, maxs, ngroups);
  if (seg) {
    const int64_t per = std::min<int64_t>(L, kSegMax);  // elements per workgroup
    const int64_t segs = cdiv(L, per);
    hipLaunchKernelGGL(quant_minmax_seg, dim3(static_cast<unsigned>(ngroups * segs)), dim3(kQuantThreads), 0, s,
                       data, L, per, segs, mins, maxs);
  } else if (n > 0) {
    hipLaunchKernelGGL(quant_minmax, dim3(cdiv(cdiv(n, kQuantRun), kQuantThreads)),
                       dim3(kQuantThreads), 0, s, data, n, qs, mins, maxs, groups);
  }
  hipLaunchKernelGGL(quant_params, dim3(cdiv(ngroups, 256)), dim3(256), 0, s, scales, zero_points,
                     ngroups, symmetric, qmin, qmax);
  if (seg) {
    hipLaunchKernelGGL(quant_values_seg, dim3(static_cast<unsigned>(cdiv(cdiv(n, 4), kQuantThreads))),
                       dim3(kQuantThreads), 0, s, data, static_cast<int>(n), static_cast<int>(L), scales,
                       zero_points, qmin, qmax, qvalues, groups);
  } else if (n > 0) {
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
