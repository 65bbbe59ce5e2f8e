// LayerNorm and RMSNorm backward.
//
// Reference kernels (one program per row, BLOCK_N tiles, two passes):
//   layer_norm_backward  kernels/teeny-kernels/src/nn/norm/layernorm.rs:300-482
//     xhat = (x - mean) * rstd, c1 = sum(dy g) / N, c2 = sum(dy g xhat) / N,
//     dx = rstd * g * (dy - c1 - xhat * c2), dweight += dy xhat, dbias += dy
//   rms_norm_backward    kernels/teeny-kernels/src/nn/norm/rmsnorm.rs:135-277
//     s = sum(dy g x) / N, dx = rrms * g * (dy - x rrms^2 s), dweight += dy x rrms
// The dx formulas are the reference's exactly (gamma outside the bracket:
// the true gradient of the forward when gamma == 1).  The reference updates
// dweight/dbias with an unsynchronised load-add-store in every program; here
// the column sums are deterministic and accumulate into the existing values.
//
// MI355X design (HBM-bound: read x and dy, write dx).  A persistent grid of G
// workgroups walks the rows (row r on workgroup r mod G); each thread owns
// VPT fixed 16-byte column vectors of every row, so gamma is loaded once and
// the per-column gradient partials stay in fp32 registers across rows.  The
// rows two ahead are loaded (raw, with their statistics; x and dy by
// non-temporal loads: LayerNorm backward 88.7 -> 86.3 us, RMSNorm 84.5 ->
// 80.1 us at [16384, 4096] bf16) before the current row's reductions, which
// are DPP wave sums plus one LDS exchange (one barrier per row: each
// register set has its own LDS slot).  One workgroup per CU: with the
// column sums below, LayerNorm backward 76.7 -> 72.0 us and RMSNorm 75.8 ->
// 70.4 us against two per CU (half the partials, and fewer bytes in flight,
// which stream faster here as in the forward); one per CU with one row
// ahead 76.0 / 70.8 us, three ahead 72.7 / 71.2 us; two per CU with one row
// ahead 76.8 / 75.7 us, three per CU 85.5 / 78.8 us.  At the end each
// workgroup writes its column partials to the stream workspace and one
// small pass adds them per column in a fixed order to dweight (and dbias).
// Without a large enough workspace
// the parameter gradients come from a column kernel that re-reads x and dy
// instead (no scratch, two more tensor reads).  Rows that do not fit the
// register plan (N > 8192 bf16 / 4096 fp32, N % 8 != 0, unaligned) take a
// multi-pass wave-per-row kernel for dx and the column kernel.
#include "common.hpp"

namespace teeny {

constexpr int kNbThreads = 256;
constexpr int kNbWaves = kNbThreads / 64;

template <typename T>
__device__ __forceinline__ void load_vec(const T *p, float *out) {
  constexpr int VEC = 16 / sizeof(T);
  const u32x4 raw = *reinterpret_cast<const u32x4 *>(p);
  T e[VEC];
  __builtin_memcpy(e, &raw, 16);
#pragma unroll
  for (int i = 0; i < VEC; ++i) out[i] = to_f32(e[i]);
}

template <typename T>
__device__ __forceinline__ void store_vec(T *p, const float *v) {
  constexpr int VEC = 16 / sizeof(T);
  T e[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) e[i] = from_f32<T>(v[i]);
  u32x4 raw;
  __builtin_memcpy(&raw, e, 16);
  __builtin_nontemporal_store(raw, reinterpret_cast<u32x4 *>(p));
}

// dx for rows blockIdx.x, blockIdx.x + G, ...; with PART, per-workgroup column
// partials of dweight (part_g) and dbias (part_b, LayerNorm) as fp32 [G, N].
// The next row's x and dy are loaded (raw, two register sets) before the
// current row's reductions, so each workgroup keeps two rows in flight.
template <typename T, int VPT, bool RMS, bool PART>
__global__ __launch_bounds__(kNbThreads) void norm_bwd_rows_kernel(
    const T *__restrict__ dy, const T *__restrict__ x, T *__restrict__ dx, const T *__restrict__ gamma,
    const float *__restrict__ st0, const float *__restrict__ st1, float *__restrict__ part_g,
    float *__restrict__ part_b, int64_t M, int32_t N, float inv_n) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int NS = RMS ? 1 : 2;  // row sums
  __shared__ float red[3][kNbWaves][NS];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int nv = N / VEC;
  const int64_t G = gridDim.x;
  float g[VPT][VEC], acc_g[VPT][VEC], acc_b[VPT][VEC];
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int v = j * kNbThreads + tid;
    if (v < nv) load_vec(gamma + static_cast<int64_t>(v) * VEC, g[j]);
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      if (v >= nv) g[j][i] = 0.0f;
      acc_g[j][i] = 0.0f;
      acc_b[j][i] = 0.0f;
    }
  }
  // raw 16-byte vectors of a row and its statistics: vectors past N load the
  // row's last vector and are zeroed by a select (no branch, so the arrays
  // stay in registers and the compiler's waits stay exact)
  auto load_raw = [&](int64_t row, u32x4 (&rx)[VPT], u32x4 (&rd)[VPT], float &sa, float &sb)
                      __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const int v = j * kNbThreads + tid;
      const int vc = v < nv ? v : nv - 1;
      const u32x4 tx = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(x + row * N + static_cast<int64_t>(vc) * VEC));
      const u32x4 td = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(dy + row * N + static_cast<int64_t>(vc) * VEC));
      const u32x4 z = {0u, 0u, 0u, 0u};
      rx[j] = v < nv ? tx : z;
      rd[j] = v < nv ? td : z;
    }
    sa = st0[row];
    sb = RMS ? sa : st1[row];
  };
  auto process = [&](int64_t row, const u32x4 (&rx)[VPT], const u32x4 (&rd)[VPT], float a, float rstd, int par)
                     __attribute__((always_inline)) {
    T *dxr = dx + row * N;
    float xv[VPT][VEC], dv[VPT][VEC];
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      T ex[VEC], ed[VEC];
      __builtin_memcpy(ex, &rx[j], 16);
      __builtin_memcpy(ed, &rd[j], 16);
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        xv[j][i] = to_f32(ex[i]);
        dv[j][i] = to_f32(ed[i]);
      }
    }
    // a: LayerNorm mean, RMSNorm rrms; rstd: LayerNorm rstd, RMSNorm rrms
    float s[NS];
#pragma unroll
    for (int k = 0; k < NS; ++k) s[k] = 0.0f;
#pragma unroll
    for (int j = 0; j < VPT; ++j)
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        const float dg = dv[j][i] * g[j][i];
        if constexpr (RMS) {
          s[0] += dg * xv[j][i];
        } else {
          s[0] += dg;
          s[1] += dg * ((xv[j][i] - a) * rstd);
        }
      }
#pragma unroll
    for (int k = 0; k < NS; ++k) s[k] = wave_total(s[k]);
    if (lane == 0)
#pragma unroll
      for (int k = 0; k < NS; ++k) red[par][w][k] = s[k];
    __syncthreads();
#pragma unroll
    for (int k = 0; k < NS; ++k) s[k] = red[par][0][k] + red[par][1][k] + red[par][2][k] + red[par][3][k];
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const int v = j * kNbThreads + tid;
      float o[VEC];
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        if constexpr (RMS) {
          const float scale = s[0] * inv_n;
          o[i] = rstd * g[j][i] * (dv[j][i] - xv[j][i] * (rstd * rstd) * scale);
          if constexpr (PART) acc_g[j][i] += dv[j][i] * xv[j][i] * rstd;
        } else {
          const float xhat = (xv[j][i] - a) * rstd;
          o[i] = rstd * g[j][i] * (dv[j][i] - s[0] * inv_n - xhat * (s[1] * inv_n));
          if constexpr (PART) {
            acc_g[j][i] += dv[j][i] * xhat;
            acc_b[j][i] += dv[j][i];
          }
        }
      }
      if (v < nv) store_vec(dxr + static_cast<int64_t>(v) * VEC, o);
    }
  };
  // three register sets, two rows ahead, unrolled by three so the sets
  // rotate without copies; each set has its own LDS slot (one barrier per
  // row).  Past the last row a prefetch re-reads the current row (cached, and
  // never used), so the loads need no branch.  The grid has at most M
  // workgroups.
  u32x4 xa[VPT], da[VPT], xb[VPT], db[VPT], xc[VPT], dc[VPT];
  float sa0, sa1, sb0, sb1, sc0, sc1;
  auto clamp = [&](int64_t r, int64_t cur) { return r < M ? r : cur; };
  int64_t row = blockIdx.x;
  load_raw(row, xa, da, sa0, sa1);
  load_raw(clamp(row + G, row), xb, db, sb0, sb1);
  for (; row < M; row += 3 * G) {
    const int64_t r1 = row + G, r2 = row + 2 * G;
    load_raw(clamp(r2, row), xc, dc, sc0, sc1);
    process(row, xa, da, sa0, sa1, 0);
    if (r1 >= M) break;
    load_raw(clamp(r2 + G, r1), xa, da, sa0, sa1);
    process(r1, xb, db, sb0, sb1, 1);
    if (r2 >= M) break;
    load_raw(clamp(r2 + 2 * G, r2), xb, db, sb0, sb1);
    process(r2, xc, dc, sc0, sc1, 2);
  }
  if constexpr (PART) {
    float *pg = part_g + static_cast<int64_t>(blockIdx.x) * N;
    float *pb = RMS ? nullptr : part_b + static_cast<int64_t>(blockIdx.x) * N;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const int v = j * kNbThreads + tid;
      if (v >= nv) continue;
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        pg[static_cast<int64_t>(v) * VEC + i] = acc_g[j][i];
        if constexpr (!RMS) pb[static_cast<int64_t>(v) * VEC + i] = acc_b[j][i];
      }
    }
  }
}

// Column sums of the per-workgroup partials in one deterministic pass.
// Workgroup (column block c, array a: 0 the dweight partials, 1 the dbias
// ones) is 64 row groups x 16 column quads: thread (r, j) adds rows r, r +
// 64, ... of columns 64 c + 4 j .. + 3 (one 16-byte load per row; eight
// loads in flight per batch of 512 rows, the rest one at a time), the
// 64 columns of one row being one 256-byte segment; the 64 row-group sums of
// a column are then added by a fixed two-level tree in LDS and accumulated
// into dweight or dbias.  (Single columns, 64-byte row segments: LayerNorm
// backward 79.1 against 76.8 us at [16384, 4096] bf16.  Two passes, slices
// of workgroups then the slices, ran it in 86.2 us against 81.4 us with one
// pass of single columns, RMSNorm 79.9 against 76.6 us.)
constexpr int kCsQuads = 16, kCsCols = 4 * kCsQuads, kCsGroups = 64, kCsThreads = kCsQuads * kCsGroups;
__global__ __launch_bounds__(kCsThreads) void norm_bwd_colsum(const float *__restrict__ part_g,
                                                              const float *__restrict__ part_b, int G, int N,
                                                              float *__restrict__ dweight,
                                                              float *__restrict__ dbias) {
  __shared__ f32x4 red[kCsGroups][kCsQuads];
  __shared__ f32x4 red2[kCsGroups / 4][kCsQuads];
  const int t = threadIdx.x;
  const int j = t % kCsQuads, r = t / kCsQuads;
  const int n = blockIdx.x * kCsCols + 4 * j;  // the thread's four columns n .. n + 3 (N % 4 == 0)
  const bool bias = blockIdx.y == 1;
  const float *part = bias ? part_b : part_g;
  f32x4 acc[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) acc[k] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  auto ld = [&](int g) { return *reinterpret_cast<const f32x4 *>(part + static_cast<int64_t>(g) * N + n); };
  if (n < N) {
    int g = r;
    for (; g + 7 * kCsGroups < G; g += 8 * kCsGroups) {
#pragma unroll
      for (int k = 0; k < 8; ++k) acc[k] += ld(g + k * kCsGroups);
    }
    for (; g < G; g += kCsGroups) acc[0] += ld(g);
  }
  red[r][j] = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
  __syncthreads();
  if (t < kCsGroups / 4 * kCsQuads) {
    const int q = t / kCsQuads;
    red2[q][j] = (red[4 * q][j] + red[4 * q + 1][j]) + (red[4 * q + 2][j] + red[4 * q + 3][j]);
  }
  __syncthreads();
  if (t < kCsQuads && n < N) {
    f32x4 sum = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int q = 0; q < kCsGroups / 4; ++q) sum += red2[q][j];
    float *out = (bias ? dbias : dweight) + n;
#pragma unroll
    for (int e = 0; e < 4; ++e) out[e] = out[e] + sum[e];
  }
}

// Parameter gradients without scratch: thread = column, all rows in order.
template <typename T, bool RMS>
__global__ __launch_bounds__(kNbThreads) void norm_bwd_cols_kernel(const T *__restrict__ dy,
                                                                   const T *__restrict__ x,
                                                                   const float *__restrict__ st0,
                                                                   const float *__restrict__ st1, int64_t M,
                                                                   int64_t N, float *__restrict__ dweight,
                                                                   float *__restrict__ dbias) {
  const int64_t n = static_cast<int64_t>(blockIdx.x) * kNbThreads + threadIdx.x;
  if (n >= N) return;
  float sg = 0.0f, sb = 0.0f;
  for (int64_t m = 0; m < M; ++m) {
    const float d = to_f32(dy[m * N + n]), xv = to_f32(x[m * N + n]);
    if constexpr (RMS) {
      sg += d * xv * st0[m];
    } else {
      sg += d * ((xv - st0[m]) * st1[m]);
      sb += d;
    }
  }
  if (dweight != nullptr) dweight[n] = dweight[n] + sg;
  if (!RMS && dbias != nullptr) dbias[n] = dbias[n] + sb;
}

// dx for any N and alignment: one wave per row, the reference's two passes.
template <typename T, bool RMS>
__global__ __launch_bounds__(kNbThreads) void norm_bwd_multipass_kernel(
    const T *__restrict__ dy, const T *__restrict__ x, T *__restrict__ dx, const T *__restrict__ gamma,
    const float *__restrict__ st0, const float *__restrict__ st1, int64_t M, int64_t N, float inv_n) {
  const int lane = threadIdx.x & 63;
  const int64_t nwaves = static_cast<int64_t>(gridDim.x) * kNbWaves;
  for (int64_t row = static_cast<int64_t>(blockIdx.x) * kNbWaves + (threadIdx.x >> 6); row < M; row += nwaves) {
    const T *xr = x + row * N, *dyr = dy + row * N;
    T *dxr = dx + row * N;
    const float a = st0[row], rstd = RMS ? a : st1[row];
    float s0 = 0.0f, s1 = 0.0f;
    for (int64_t c = lane; c < N; c += 64) {
      const float dg = to_f32(dyr[c]) * to_f32(gamma[c]), xv = to_f32(xr[c]);
      if constexpr (RMS) {
        s0 += dg * xv;
      } else {
        s0 += dg;
        s1 += dg * ((xv - a) * rstd);
      }
    }
    s0 = wave_sum(s0);
    s1 = wave_sum(s1);
    for (int64_t c = lane; c < N; c += 64) {
      const float d = to_f32(dyr[c]), gm = to_f32(gamma[c]), xv = to_f32(xr[c]);
      float o;
      if constexpr (RMS) o = rstd * gm * (d - xv * (rstd * rstd) * (s0 * inv_n));
      else o = rstd * gm * (d - s0 * inv_n - ((xv - a) * rstd) * (s1 * inv_n));
      dxr[c] = from_f32<T>(o);
    }
  }
}

// Workgroups of the row kernel: one per CU, at most one per row.
static int bwd_groups(int64_t M) {
  return static_cast<int>(std::min<int64_t>(M, static_cast<int64_t>(device_cu_count())));
}

template <typename T>
static int bwd_vpt(int64_t N, bool vec_ok) {
  constexpr int VEC = 16 / sizeof(T);
  if (!vec_ok || N % VEC != 0) return 0;
  const int64_t nv = N / VEC;
  for (int v : {1, 2, 4})
    if (nv <= static_cast<int64_t>(v) * kNbThreads) return v;
  return 0;
}

// [part_g G x N][part_b G x N], fp32
static size_t bwd_scratch_bytes(int64_t M, int64_t N, bool rms) {
  return static_cast<size_t>(bwd_groups(M)) * static_cast<size_t>(N) * 4 * (rms ? 1 : 2);
}

template <typename T, int VPT, bool RMS, bool PART>
static void launch_bwd_rows(const void *dy, const void *x, void *dx, const void *g, const float *st0,
                            const float *st1, float *pg, float *pb, int64_t M, int64_t N, int G, hipStream_t s) {
  hipLaunchKernelGGL((norm_bwd_rows_kernel<T, VPT, RMS, PART>), dim3(G), dim3(kNbThreads), 0, s,
                     static_cast<const T *>(dy), static_cast<const T *>(x), static_cast<T *>(dx),
                     static_cast<const T *>(g), st0, st1, pg, pb, M, static_cast<int32_t>(N),
                     1.0f / static_cast<float>(N));
}

template <typename T, bool RMS>
static teeny_status norm_bwd(const void *dy, const void *x, void *dx, const void *g, const float *st0,
                             const float *st1, float *dweight, float *dbias, int64_t M, int64_t N, hipStream_t s,
                             const char *name) {
  const bool vec_ok = aligned(dy, 16) && aligned(x, 16) && aligned(dx, 16) && aligned(g, 16);
  const int vpt = bwd_vpt<T>(N, vec_ok);
  const bool grads = dweight != nullptr || (!RMS && dbias != nullptr);
  const int G = bwd_groups(M);
  const Scratch scr = stream_scratch(s);
  const bool part = grads && vpt > 0 && scr.ptr != nullptr && aligned(scr.ptr, 16) &&
                    scr.bytes >= bwd_scratch_bytes(M, N, RMS);
  float *pg = part ? static_cast<float *>(scr.ptr) : nullptr;
  float *pb = part && !RMS ? pg + static_cast<int64_t>(G) * N : nullptr;
  if (vpt > 0) {
#define TEENY_NB_ROWS(V)                                                                            \
  do {                                                                                              \
    if (part) launch_bwd_rows<T, V, RMS, true>(dy, x, dx, g, st0, st1, pg, pb, M, N, G, s);         \
    else launch_bwd_rows<T, V, RMS, false>(dy, x, dx, g, st0, st1, nullptr, nullptr, M, N, G, s);   \
  } while (0)
    switch (vpt) {
      case 1: TEENY_NB_ROWS(1); break;
      case 2: TEENY_NB_ROWS(2); break;
      case 4: TEENY_NB_ROWS(4); break;
      default: TEENY_NB_ROWS(4); break;
    }
#undef TEENY_NB_ROWS
  } else {
    const int blocks = static_cast<int>(std::min<int64_t>(cdiv(M, kNbWaves), 8 * device_cu_count()));
    hipLaunchKernelGGL((norm_bwd_multipass_kernel<T, RMS>), dim3(blocks), dim3(kNbThreads), 0, s,
                       static_cast<const T *>(dy), static_cast<const T *>(x), static_cast<T *>(dx),
                       static_cast<const T *>(g), st0, st1, M, N, 1.0f / static_cast<float>(N));
  }
  teeny_status st = after_launch(name, s);
  if (st != TEENY_OK || !grads) return st;
  if (part) {
    // one column-sum grid row per requested gradient (dweight, dbias)
    const bool want_g = dweight != nullptr, want_b = !RMS && dbias != nullptr;
    const float *src0 = want_g ? pg : pb;
    float *dst0 = want_g ? dweight : dbias;
    hipLaunchKernelGGL(norm_bwd_colsum, dim3(static_cast<unsigned>(cdiv(N, kCsCols)), want_g && want_b ? 2u : 1u),
                       dim3(kCsThreads), 0, s, src0, pb, G, static_cast<int>(N), dst0, dbias);
  } else {
    hipLaunchKernelGGL((norm_bwd_cols_kernel<T, RMS>), dim3(static_cast<unsigned>(cdiv(N, kNbThreads))),
                       dim3(kNbThreads), 0, s, static_cast<const T *>(dy), static_cast<const T *>(x), st0, st1, M,
                       N, dweight, RMS ? nullptr : dbias);
  }
  return after_launch(name, s);
}

static teeny_status norm_bwd_entry(const void *dy, const void *x, void *dx, const void *g, float *dweight,
                                   float *dbias, const float *st0, const float *st1, int64_t M, int64_t N,
                                   bool rms, teeny_dtype dtype, teeny_stream stream, const char *name) {
  const std::string nm(name);
  TEENY_REQUIRE(M >= 0 && N >= 0, TEENY_ERR_SHAPE_MISMATCH, nm + ": negative M or N");
  if (M == 0) return TEENY_OK;
  TEENY_REQUIRE(N > 0 && N <= 0x7fffffff, TEENY_ERR_SHAPE_MISMATCH, nm + ": N must be in [1, 2^31)");
  TEENY_REQUIRE(dy != nullptr && x != nullptr && dx != nullptr && g != nullptr && st0 != nullptr &&
                    (rms || st1 != nullptr),
                TEENY_ERR_NULL_POINTER, nm + (rms ? ": dy/x/dx/weight/rrms" : ": dy/x/dx/weight/mean/rstd"));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == TEENY_F32)
    return rms ? norm_bwd<float, true>(dy, x, dx, g, st0, st1, dweight, dbias, M, N, s, name)
               : norm_bwd<float, false>(dy, x, dx, g, st0, st1, dweight, dbias, M, N, s, name);
  if (dtype == TEENY_BF16)
    return rms ? norm_bwd<bf16, true>(dy, x, dx, g, st0, st1, dweight, dbias, M, N, s, name)
               : norm_bwd<bf16, false>(dy, x, dx, g, st0, st1, dweight, dbias, M, N, s, name);
  return fail(TEENY_ERR_UNSUPPORTED_DTYPE, nm + ": dtype must be F32 or BF16");
}

}  // namespace teeny

using namespace teeny;

extern "C" {

teeny_status teeny_layer_norm_backward(const void *dy, const void *x, void *dx, const void *weight,
                                       float *dweight, float *dbias, const float *mean, const float *rstd,
                                       int64_t M, int64_t N, teeny_dtype dtype, teeny_stream stream) {
  return norm_bwd_entry(dy, x, dx, weight, dweight, dbias, mean, rstd, M, N, false, dtype, stream,
                        "layer_norm_backward");
}

teeny_status teeny_rms_norm_backward(const void *dy, const void *x, void *dx, const void *weight, float *dweight,
                                     const float *rrms, int64_t M, int64_t N, teeny_dtype dtype,
                                     teeny_stream stream) {
  return norm_bwd_entry(dy, x, dx, weight, dweight, nullptr, rrms, nullptr, M, N, true, dtype, stream,
                        "rms_norm_backward");
}

teeny_status teeny_norm_backward_workspace_size(int64_t M, int64_t N, int32_t is_rms, teeny_dtype dtype,
                                                size_t *bytes) {
  TEENY_REQUIRE(bytes != nullptr, TEENY_ERR_NULL_POINTER, "norm_backward_workspace_size: bytes");
  *bytes = 0;
  TEENY_REQUIRE(M >= 0 && N >= 0, TEENY_ERR_SHAPE_MISMATCH, "norm_backward_workspace_size: negative size");
  TEENY_REQUIRE(dtype == TEENY_F32 || dtype == TEENY_BF16, TEENY_ERR_UNSUPPORTED_DTYPE,
                "norm_backward_workspace_size: dtype must be F32 or BF16");
  if (M == 0 || N == 0) return TEENY_OK;
  // the row kernel's plan (aligned operands assumed); other shapes use no scratch
  const int vpt = dtype == TEENY_F32 ? bwd_vpt<float>(N, true) : bwd_vpt<bf16>(N, true);
  if (vpt > 0) *bytes = bwd_scratch_bytes(M, N, is_rms != 0);
  return TEENY_OK;
}

}  // extern "C"
