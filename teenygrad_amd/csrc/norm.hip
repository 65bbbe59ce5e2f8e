// LayerNorm (inference) and RMSNorm over the last dimension of [M, N].
//
// Reference kernels (one program per row, BLOCK_N-wide tiles):
//   layer_norm_forward_inference  kernels/teeny-kernels/src/nn/norm/layernorm.rs:42-157
//     three passes over the row: mean (:61-77), variance of (x - mean) (:79-100),
//     normalise + affine (:102-156).
//   rms_norm_forward              kernels/teeny-kernels/src/nn/norm/rmsnorm.rs:39-119
//     two passes: sum of squares (:58-79) and rrms store (:80-83), normalise (:85-118).
//
// MI355X design: a row is held in registers across WPR waves of one
// workgroup (each lane VPL 16-byte vectors, VEC = 8 bf16 or 4 fp32), so x is
// read from HBM exactly once and y written once — the reference's four
// tensor passes become the two-pass minimum, with the same two-pass
// mean/variance arithmetic done on registers.  Per-row sums are a DPP wave
// reduction plus one LDS exchange between the row's waves (one barrier per
// statistic).  Lane l of wave p of a row loads columns
// ((p*VPL + j)*64 + l)*VEC, so each load instruction is one contiguous 1 KiB
// request.  For N = 4096 bf16 this is 2 waves per row (two rows per
// workgroup) and 4 vectors per lane, which keeps enough 16-byte loads in
// flight to stream at about the chip's copy rate; gamma/beta (L2-resident,
// 8 KiB) are loaded right after x, ahead of the reductions.  Outputs use
// ordinary stores, so that the activation that follows a norm finds them in
// the Infinity Cache (non-temporal stores: the LayerNorm -> GELU, SiLU;
// RMSNorm -> GELU, SiLU chain 6690 -> 6370 GB/s, the norms alone within
// 3 %).  RMSNorm reads x by non-temporal loads; LayerNorm
// keeps temporal ones: non-temporal loads made a LayerNorm on cold data 2 %
// faster (47.9 -> 46.8 us) but the chain of LayerNorm, GELU, SiLU and
// RMSNorm over one X 2 % slower (the RMSNorm re-reads X, part of it from the
// Infinity Cache), while in RMSNorm alone they take the chain from 6281 to
// 6370 GB/s.  Longer
// rows, unaligned pointers or N % VEC != 0 take a multi-pass kernel with the
// reference's pass structure.
#include "common.hpp"

namespace teeny {

constexpr int kNormThreads = 256;
constexpr int kNormWaves = kNormThreads / 64;
constexpr int kNormMaxBlocks = 256 * 8;

template <typename T, int WPR, int VPL, bool RMS, int ACT>
__global__ __launch_bounds__(kNormThreads) void norm_rows_kernel(
    const T *__restrict__ x, T *__restrict__ y, const T *__restrict__ gamma,
    const T *__restrict__ beta, float *__restrict__ st0, float *__restrict__ st1, int64_t M, int32_t N, float eps,
    float inv_n) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int RPB = kNormWaves / WPR;  // rows per workgroup
  constexpr bool fast = !std::is_same<T, float>::value;
  __shared__ float red[kNormWaves][2];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int rsub = w / WPR, part = w % WPR;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * RPB + rsub;
  const bool row_ok = row < M;
  const T *xr = x + (row_ok ? row : 0) * N;
  T *yr = y + (row_ok ? row : 0) * N;

  u32x4 raw[VPL];
  bool valid[VPL];
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int col = ((part * VPL + j) * 64 + lane) * VEC;
    valid[j] = row_ok && col < N;
    const u32x4 *src = reinterpret_cast<const u32x4 *>(xr + col);
    raw[j] = valid[j] ? (RMS ? __builtin_nontemporal_load(src) : *src) : u32x4{0u, 0u, 0u, 0u};
  }
  // gamma / beta are issued right behind x, so their (L2) latency overlaps
  // the row's reductions instead of following them
  u32x4 rg[VPL], rbt[VPL];
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int col = ((part * VPL + j) * 64 + lane) * VEC;
    rg[j] = valid[j] ? *reinterpret_cast<const u32x4 *>(gamma + col) : u32x4{0u, 0u, 0u, 0u};
    if constexpr (!RMS) rbt[j] = valid[j] ? *reinterpret_cast<const u32x4 *>(beta + col) : u32x4{0u, 0u, 0u, 0u};
  }
  float v[VPL][VEC];
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    T e[VEC];
    __builtin_memcpy(e, &raw[j], 16);
#pragma unroll
    for (int i = 0; i < VEC; ++i) v[j][i] = to_f32(e[i]);  // invalid vectors hold zeros
  }

  // row total of a per-lane partial: wave shuffle, then across the row's waves via LDS
  auto row_sum = [&](float part_sum, int slot) {
    part_sum = wave_total(part_sum);
    if (WPR == 1) return part_sum;
    if (lane == 0) red[w][slot] = part_sum;
    __syncthreads();
    float t = 0.0f;
#pragma unroll
    for (int p = 0; p < WPR; ++p) t += red[rsub * WPR + p][slot];
    return t;
  };

  float mean = 0.0f, rstd;
  if constexpr (RMS) {
    float q = 0.0f;
#pragma unroll
    for (int j = 0; j < VPL; ++j)
#pragma unroll
      for (int i = 0; i < VEC; ++i) q += v[j][i] * v[j][i];
    q = row_sum(q, 0);
    rstd = rsqrtf(q * inv_n + eps);
    if (st0 != nullptr && row_ok && part == 0 && lane == 0) st0[row] = rstd;  // rrms
  } else {
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < VPL; ++j)
#pragma unroll
      for (int i = 0; i < VEC; ++i) s += v[j][i];
    mean = row_sum(s, 0) * inv_n;
    float q = 0.0f;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      if (valid[j]) {
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
          const float d = v[j][i] - mean;
          q += d * d;
        }
      }
    }
    rstd = rsqrtf(row_sum(q, 1) * inv_n + eps);
    if (row_ok && part == 0 && lane == 0) {  // training forward: saved statistics
      if (st0 != nullptr) st0[row] = mean;
      if (st1 != nullptr) st1[row] = rstd;
    }
  }

#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    if (!valid[j]) continue;
    const int col = ((part * VPL + j) * 64 + lane) * VEC;
    T ge[VEC], be[VEC];
    __builtin_memcpy(ge, &rg[j], 16);
    if constexpr (!RMS) __builtin_memcpy(be, &rbt[j], 16);
    T e[VEC];
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      const float o = RMS ? v[j][i] * rstd * to_f32(ge[i])
                          : (v[j][i] - mean) * rstd * to_f32(ge[i]) + to_f32(be[i]);
      e[i] = from_f32<T>(apply_act<ACT, fast>(o));
    }
    u32x4 r;
    __builtin_memcpy(&r, e, 16);
    *reinterpret_cast<u32x4 *>(yr + col) = r;
  }
}

// Any N, any alignment: the reference's multi-pass structure, one wave per row.
template <typename T, bool RMS, int ACT>
__global__ __launch_bounds__(kNormThreads) void norm_multipass_kernel(
    const T *__restrict__ x, T *__restrict__ y, const T *__restrict__ gamma,
    const T *__restrict__ beta, float *__restrict__ st0, float *__restrict__ st1, int64_t M, int64_t N, float eps,
    float inv_n) {
  constexpr bool fast = !std::is_same<T, float>::value;
  const int lane = threadIdx.x & 63;
  const int64_t nwaves = static_cast<int64_t>(gridDim.x) * kNormWaves;
  for (int64_t row = static_cast<int64_t>(blockIdx.x) * kNormWaves + (threadIdx.x >> 6); row < M;
       row += nwaves) {
    const T *xr = x + row * N;
    T *yr = y + row * N;
    float mean = 0.0f, rstd;
    if constexpr (RMS) {
      float q = 0.0f;
      for (int64_t c = lane; c < N; c += 64) {
        float v = to_f32(xr[c]);
        q += v * v;
      }
      q = wave_sum(q);
      rstd = rsqrtf(q * inv_n + eps);
      if (st0 != nullptr && lane == 0) st0[row] = rstd;  // rrms
    } else {
      float s = 0.0f;
      for (int64_t c = lane; c < N; c += 64) s += to_f32(xr[c]);
      s = wave_sum(s);
      mean = s * inv_n;
      float q = 0.0f;
      for (int64_t c = lane; c < N; c += 64) {
        float d = to_f32(xr[c]) - mean;
        q += d * d;
      }
      q = wave_sum(q);
      rstd = rsqrtf(q * inv_n + eps);
      if (lane == 0) {
        if (st0 != nullptr) st0[row] = mean;
        if (st1 != nullptr) st1[row] = rstd;
      }
    }
    for (int64_t c = lane; c < N; c += 64) {
      float v = to_f32(xr[c]);
      float o = RMS ? v * rstd * to_f32(gamma[c])
                    : (v - mean) * rstd * to_f32(gamma[c]) + to_f32(beta[c]);
      yr[c] = from_f32<T>(apply_act<ACT, fast>(o));
    }
  }
}

// Dynamic LDS that no kernel touches, sized so that at most `wgs` workgroups
// fit in one CU's 160 KiB (0: no cap).  Used as an occupancy cap where fewer
// resident rows stream faster.
static unsigned occupancy_cap_lds(int wgs) { return wgs > 0 ? 160u * 1024u / (wgs + 1) + 1024u : 0u; }

template <typename T, int WPR, int VPL, bool RMS, int ACT>
static void launch_rows(const void *x, void *y, const void *g, const void *b, float *st0, float *st1,
                        int64_t M, int64_t N, float eps, float inv_n, hipStream_t s, int wgs_per_cu = 0) {
  constexpr int RPB = kNormWaves / WPR;
  hipLaunchKernelGGL((norm_rows_kernel<T, WPR, VPL, RMS, ACT>), dim3(cdiv(M, RPB)),
                     dim3(kNormThreads), occupancy_cap_lds(wgs_per_cu), s, static_cast<const T *>(x), static_cast<T *>(y),
                     static_cast<const T *>(g), static_cast<const T *>(b), st0, st1, M,
                     static_cast<int32_t>(N), eps, inv_n);
}

template <typename T, bool RMS, int ACT>
static teeny_status launch_norm(const void *x, void *y, const void *g, const void *b, float *st0, float *st1,
                                int64_t M, int64_t N, float eps, hipStream_t s, const char *name) {
  constexpr int VEC = 16 / sizeof(T);
  const float inv_n = 1.0f / static_cast<float>(N);
  const bool vec_ok = (N % VEC == 0) && aligned(x, 16) && aligned(y, 16) && aligned(g, 16) &&
                      (RMS || aligned(b, 16));
  const int64_t nv = N / VEC;  // 16-byte vectors per row
  TEENY_REQUIRE(cdiv(M, 4) <= 0x7fffffff, TEENY_ERR_SHAPE_MISMATCH, std::string(name) + ": M too large");
  if (vec_ok && nv <= 64) {
    launch_rows<T, 1, 1, RMS, ACT>(x, y, g, b, st0, st1, M, N, eps, inv_n, s);
  } else if (vec_ok && nv <= 128) {
    launch_rows<T, 2, 1, RMS, ACT>(x, y, g, b, st0, st1, M, N, eps, inv_n, s);
  } else if (vec_ok && nv <= 256) {
    launch_rows<T, 4, 1, RMS, ACT>(x, y, g, b, st0, st1, M, N, eps, inv_n, s);
  } else if (vec_ok && nv <= 512) {
    // two waves per row, two rows per workgroup: measured against four waves
    // per row at [16384, 4096] bf16, LayerNorm 47.3 vs 50.1 us, RMSNorm equal.
    // At most four workgroups per CU (registers alone allow five): LayerNorm
    // 47.7 -> 46.4 us, RMSNorm 45.9 -> 45.0 us; three per CU 47.8 / 45.9 us,
    // two 52 / 48 us.
    launch_rows<T, 2, 4, RMS, ACT>(x, y, g, b, st0, st1, M, N, eps, inv_n, s, 4);
  } else if (vec_ok && nv <= 1024) {
    launch_rows<T, 4, 4, RMS, ACT>(x, y, g, b, st0, st1, M, N, eps, inv_n, s);
  } else if (vec_ok && nv <= 2048) {
    launch_rows<T, 4, 8, RMS, ACT>(x, y, g, b, st0, st1, M, N, eps, inv_n, s);
  } else {
    const int blocks = static_cast<int>(std::min<int64_t>(cdiv(M, kNormWaves), kNormMaxBlocks));
    hipLaunchKernelGGL((norm_multipass_kernel<T, RMS, ACT>), dim3(blocks), dim3(kNormThreads), 0,
                       s, static_cast<const T *>(x), static_cast<T *>(y),
                       static_cast<const T *>(g), static_cast<const T *>(b), st0, st1, M, N, eps,
                       inv_n);
  }
  return after_launch(name, s);
}

template <typename T, bool RMS>
static teeny_status dispatch_act(const void *x, void *y, const void *g, const void *b, float *st0, float *st1,
                                 int64_t M, int64_t N, float eps, int act, hipStream_t s,
                                 const char *name) {
  switch (act) {
    case TEENY_ACT_NONE: return launch_norm<T, RMS, TEENY_ACT_NONE>(x, y, g, b, st0, st1, M, N, eps, s, name);
    case TEENY_ACT_RELU: return launch_norm<T, RMS, TEENY_ACT_RELU>(x, y, g, b, st0, st1, M, N, eps, s, name);
    case TEENY_ACT_GELU_TANH: return launch_norm<T, RMS, TEENY_ACT_GELU_TANH>(x, y, g, b, st0, st1, M, N, eps, s, name);
    case TEENY_ACT_SILU: return launch_norm<T, RMS, TEENY_ACT_SILU>(x, y, g, b, st0, st1, M, N, eps, s, name);
    default: return fail(TEENY_ERR_INVALID_ARGUMENT, std::string(name) + ": unknown activation");
  }
}

static teeny_status norm_entry(const void *x, void *y, const void *g, const void *b, float *st0, float *st1,
                               int64_t M, int64_t N, float eps, bool rms, int act,
                               teeny_dtype dtype, teeny_stream stream, const char *name) {
  const std::string n(name);
  TEENY_REQUIRE(M >= 0 && N >= 0, TEENY_ERR_SHAPE_MISMATCH, n + ": negative M or N");
  if (M == 0) return TEENY_OK;
  TEENY_REQUIRE(N > 0, TEENY_ERR_SHAPE_MISMATCH, n + ": N must be positive");
  TEENY_REQUIRE(N <= 0x7fffffff, TEENY_ERR_SHAPE_MISMATCH, n + ": N exceeds 2^31-1");
  TEENY_REQUIRE(x != nullptr && y != nullptr && g != nullptr, TEENY_ERR_NULL_POINTER,
                n + ": x/y/weight");
  TEENY_REQUIRE(rms || b != nullptr, TEENY_ERR_NULL_POINTER, n + ": bias");
  TEENY_REQUIRE(act >= TEENY_ACT_NONE && act <= TEENY_ACT_SILU, TEENY_ERR_INVALID_ARGUMENT,
                n + ": unknown activation");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == TEENY_F32) {
    return rms ? dispatch_act<float, true>(x, y, g, b, st0, st1, M, N, eps, act, s, name)
               : dispatch_act<float, false>(x, y, g, b, st0, st1, M, N, eps, act, s, name);
  }
  if (dtype == TEENY_BF16) {
    return rms ? dispatch_act<bf16, true>(x, y, g, b, st0, st1, M, N, eps, act, s, name)
               : dispatch_act<bf16, false>(x, y, g, b, st0, st1, M, N, eps, act, s, name);
  }
  return fail(TEENY_ERR_UNSUPPORTED_DTYPE, n + ": dtype must be F32 or BF16");
}

}  // namespace teeny

using namespace teeny;

extern "C" {

teeny_status teeny_layer_norm_forward_inference(const void *x, void *y, const void *weight,
                                                const void *bias, int64_t M, int64_t N,
                                                float eps, teeny_dtype dtype,
                                                teeny_stream stream) {
  return norm_entry(x, y, weight, bias, nullptr, nullptr, M, N, eps, false, TEENY_ACT_NONE, dtype, stream,
                    "layer_norm_forward_inference");
}

teeny_status teeny_rms_norm_forward(const void *x, void *y, const void *weight, float *rrms,
                                    int64_t M, int64_t N, float eps, teeny_dtype dtype,
                                    teeny_stream stream) {
  return norm_entry(x, y, weight, nullptr, rrms, nullptr, M, N, eps, true, TEENY_ACT_NONE, dtype, stream,
                    "rms_norm_forward");
}

teeny_status teeny_layer_norm_forward(const void *x, void *y, const void *weight, const void *bias,
                                      float *mean, float *rstd, int64_t M, int64_t N, float eps,
                                      teeny_dtype dtype, teeny_stream stream) {
  TEENY_REQUIRE(M == 0 || (mean != nullptr && rstd != nullptr), TEENY_ERR_NULL_POINTER,
                "layer_norm_forward: mean/rstd");
  return norm_entry(x, y, weight, bias, mean, rstd, M, N, eps, false, TEENY_ACT_NONE, dtype, stream,
                    "layer_norm_forward");
}

teeny_status teeny_norm_act_forward(const void *x, void *y, const void *weight, const void *bias,
                                    int64_t M, int64_t N, float eps, int32_t is_rms,
                                    teeny_activation act, teeny_dtype dtype, teeny_stream stream) {
  return norm_entry(x, y, weight, bias, nullptr, nullptr, M, N, eps, is_rms != 0, act, dtype, stream,
                    "norm_act_forward");
}

}  // extern "C"
