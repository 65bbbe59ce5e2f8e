// MFMA GEMM core shared by the linear (bf16 and W8A16) and NHWC implicit-GEMM
// conv2d kernels.
//
//   C[m, n] = act( scale[n] * sum_k A[m, k] * B[n, k] + bias[n] )
//
// A is bf16 and K-contiguous: either a plain row-major matrix (linear, 1x1
// stride-1 conv) or gathered on the fly from an NHWC activation (implicit
// GEMM: m = (b, oh, ow), k = (kh, kw, ci), zero padding by predicate).
// B is [N, K] K-contiguous, bf16 or int8; int8 is converted to bf16 (exact:
// |q| <= 128 fits bf16's 8-bit significand) while staging into LDS, so the
// dequant of teeny-quant's dequantize_affine (affine.rs:151-161) costs no
// HBM traffic and its per-channel scale is applied to the fp32 accumulator.
//
// Tiling: BM x BN x 64 per workgroup of 256 threads (4 waves as WAVES_M x
// WAVES_N), each wave a (BM/WAVES_M) x (BN/WAVES_N) block of
// v_mfma_f32_32x32x16_bf16 tiles.  Large tiles (256 x 256, 128 x 128 per
// wave, accumulators in AGPRs, one workgroup per CU) need 0.5 KiB of LDS
// fragment reads per MFMA; 128 x 128 tiles need 1 KiB, which is the LDS
// bandwidth limit, so the launcher picks the largest tile that still fills
// the chip.  The MFMA computes C^T (weights as the A operand, activations as
// the B operand) so each lane's accumulator column is one output row m and
// four consecutive registers are four consecutive n: the epilogue writes
// 8-byte bf16x4 stores.  LDS rows are padded to 72 elements (144 B), which
// makes the 16-byte fragment reads of 16 consecutive rows hit 16 disjoint
// bank quads.  Two LDS stages: the next k-tile is fetched into registers
// before the current one is consumed and written to the other stage
// afterwards, so one barrier per k-tile suffices; within a k-tile the
// fragments of step s+1 are read before the MFMAs of step s issue.
// Workgroups are remapped so that each XCD (8 per chip, workgroups dealt
// round-robin) receives a contiguous run of tiles, which share B tiles in
// that XCD's L2.
#pragma once

#include <algorithm>

#include "mfma.hpp"

namespace teeny {

enum GemmAMode : int {
  kAPlain = 0,     // A[m*lda + k]
  kAConvVec = 1,   // NHWC gather, C_IN % 8 == 0 (16-byte chunks never straddle a tap)
  kAConvScalar = 2 // NHWC gather, any C_IN (element-wise)
};

struct GemmParams {
  const bf16 *A;
  int64_t lda;
  const void *B;  // bf16 or int8, [N][ldb]
  int64_t ldb;
  bf16 *C;
  int64_t ldc;
  const float *scale;  // [N] or null
  const float *bias;   // [N] or null (fp32)
  const bf16 *bias_bf16;  // [N] or null
  int M, N, K;
  int act;  // teeny_activation applied in the epilogue
  // implicit-GEMM conv geometry (NHWC)
  int H, W, Cin, OH, OW, KH, KW, SH, SW, PH, PW;
  // split-K: when ws is set, workgroup (tile, split) multiplies k-tiles
  // [split * kt_split, (split + 1) * kt_split) and stores its raw fp32
  // partial tile to ws[split][m][n]; gemm_splitk_finalize sums the splits
  // and applies the epilogue.
  float *ws;
  int kt_split;
  // byte extents of A and B (each below 2^31: the vector loads address them
  // through buffer resources with 32-bit offsets; larger problems are split
  // on the host)
  int a_bytes, b_bytes;
  // grid order: consecutive tiles (one XCD's run, one L2) walk along N and
  // share their A row block (1), or walk along M and share B (0)
  int n_fast;
  // LDS-DMA kernel only: when > 0, consecutive tiles first cover `group`
  // tiles of the other dimension (a group x run block of tiles per XCD, so
  // both operands are shared through its L2), then step along n_fast's
  // dimension
  int group;
  // Output rows remapped (the sub-pixel phases of a strided conv's dx, whose
  // rows are every SH-th row and SW-th column of dx): when c_ow > 0, row
  // m = (b, u, v) with v = m % c_ow, u = (m / c_ow) % c_oh starts at element
  // b c_sb + u c_su + v c_sv of C, and ldc is unused.  Only the
  // register-staged kernels and the split-K finalize take it.
  int c_ow, c_oh;
  int64_t c_sb, c_su, c_sv;
  // Grouped conv (groups > 1; register-staged kernels only): workgroup row
  // blockIdx.y is group g, whose A, B and C start g g_a, g g_b and g g_c
  // elements in and whose scale / bias start g N in; cst is the pixel
  // stride of the NHWC gather (all the image's channels; 0: Cin).
  int groups, cst;
  int64_t g_a, g_b, g_c;
};

// Element offset of output row m in C (see GemmParams::c_ow).
__device__ __forceinline__ int64_t c_row(const GemmParams &p, int m) {
  if (p.c_ow <= 0) return static_cast<int64_t>(m) * p.ldc;
  const int v = m % p.c_ow, t = m / p.c_ow;
  return (t / p.c_oh) * p.c_sb + (t % p.c_oh) * p.c_su + v * p.c_sv;
}
// Whether every output row starts 16-byte aligned (8 bf16).
__host__ __device__ inline bool c_rows_vec16(const GemmParams &p) {
  const bool strides = p.c_ow > 0 ? (p.c_sb % 8 == 0 && p.c_su % 8 == 0 && p.c_sv % 8 == 0) : (p.ldc % 8 == 0);
  return strides && (reinterpret_cast<uintptr_t>(p.C) & 15) == 0;
}


__device__ __forceinline__ void epi_coeffs(const GemmParams &p, int n, float (&mul)[4], float (&add)[4]) {
  if (n + 4 <= p.N && (n & 3) == 0) {
    // four in-range columns: vector loads (n % 4 == 0 keeps them aligned)
    f32x4 m4 = {1.0f, 1.0f, 1.0f, 1.0f}, a4 = {0.0f, 0.0f, 0.0f, 0.0f};
    if (p.scale != nullptr && (reinterpret_cast<uintptr_t>(p.scale) & 15) == 0)
      m4 = *reinterpret_cast<const f32x4 *>(p.scale + n);
    else if (p.scale != nullptr)
      for (int e = 0; e < 4; ++e) m4[e] = p.scale[n + e];
    if (p.bias != nullptr && (reinterpret_cast<uintptr_t>(p.bias) & 15) == 0)
      a4 = *reinterpret_cast<const f32x4 *>(p.bias + n);
    else if (p.bias != nullptr)
      for (int e = 0; e < 4; ++e) a4[e] = p.bias[n + e];
    if (p.bias_bf16 != nullptr) {
      bf16x4 b4;
      if ((reinterpret_cast<uintptr_t>(p.bias_bf16) & 7) == 0) {
        b4 = *reinterpret_cast<const bf16x4 *>(p.bias_bf16 + n);
      } else {
        for (int e = 0; e < 4; ++e) b4[e] = p.bias_bf16[n + e];
      }
      for (int e = 0; e < 4; ++e) a4[e] += static_cast<float>(b4[e]);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      mul[e] = m4[e];
      add[e] = a4[e];
    }
    return;
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int ne = n + e;
    float m = 1.0f, a = 0.0f;
    if (ne < p.N) {
      if (p.scale != nullptr) m = p.scale[ne];
      if (p.bias != nullptr) a = p.bias[ne];
      if (p.bias_bf16 != nullptr) a += static_cast<float>(p.bias_bf16[ne]);
    }
    mul[e] = m;
    add[e] = a;
  }
}

// ── epilogue helpers ─────────────────────────────────────────────────────
// y = act(acc * mul[n] + add[n]) with mul = scale (or 1) and add = bias
// (fp32 or bf16, or 0).  The activation is applied branch-free per element:
// GELU-tanh and SiLU share y = r / (1 + 2^(r * (k1 + k3 r^2))) (GELU:
// k1 = -2 sqrt(2/pi) log2 e, k3 = 0.044715 k1; SiLU: k1 = -log2 e, k3 = 0),
// behind one wave-uniform branch for the whole tile, and ReLU is a clamp
// that keeps NaN (x < 0 ? 0 : x).  Same functions as act_gelu<true> /
// act_silu<true> / act_relu.
struct EpiAct {
  float k1, k3;
  bool sig, relu;
};
__device__ __forceinline__ EpiAct epi_act(int act) {
  constexpr float kL2e = 1.4426950408889634f;
  EpiAct a{0.0f, 0.0f, false, act == TEENY_ACT_RELU};
  if (act == TEENY_ACT_GELU_TANH) {
    a.k1 = -1.5957691216057308f * kL2e;
    a.k3 = a.k1 * 0.044715f;
    a.sig = true;
  } else if (act == TEENY_ACT_SILU) {
    a.k1 = -kL2e;
    a.sig = true;
  }
  return a;
}
__device__ __forceinline__ float epi_sig(float r, const EpiAct &a) {
  return r * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(r * __builtin_fmaf(a.k3, r * r, a.k1)));
}
// mul / add for the four consecutive columns n .. n+3 (columns past N: 1 / 0)
template <int BM, int BN>
constexpr int gemm_min_waves() {
  return (BM * BN >= 256 * 128) ? 1 : 2;
}

// BK: k-tile depth (32 or 64).  PF: global->register prefetch depth in k-tiles (1 or 2).
template <int BM, int BN, int BK, int WAVES_M, int PF, bool INT8B, int AMODE, bool KVEC = true>
__global__ __launch_bounds__(256, (gemm_min_waves<BM, BN>())) void gemm_mfma_kernel(GemmParams p0) {
  GemmParams p = p0;
  if (p0.groups > 1) {
    const int grp = static_cast<int>(blockIdx.y);
    constexpr int ES = INT8B ? 1 : 2;
    p.A += grp * p0.g_a;
    p.a_bytes -= static_cast<int>(grp * p0.g_a * 2);
    p.B = static_cast<const char *>(p0.B) + grp * p0.g_b * ES;
    p.b_bytes -= static_cast<int>(grp * p0.g_b * ES);
    p.C += grp * p0.g_c;
    if (p.scale != nullptr) p.scale += static_cast<int64_t>(grp) * p0.N;
    if (p.bias != nullptr) p.bias += static_cast<int64_t>(grp) * p0.N;
    if (p.bias_bf16 != nullptr) p.bias_bf16 += static_cast<int64_t>(grp) * p0.N;
  }
  const int cst = p.cst > 0 ? p.cst : p.Cin;  // NHWC pixel stride (elements)
  // LDS rows.  k-depth 64: padded to 72 elements.  k-depth 32: dense
  // 32-element (64-byte) rows whose 16-byte chunk c sits at position
  // c ^ ((row >> 2) & 3), so that both the row-chunk stores (16 lanes: 4
  // rows x 4 chunks) and the fragment reads (16 lanes: 16 rows, one chunk)
  // cover distinct banks (80-byte padded rows cost 2-way store conflicts).
  constexpr bool SWZ = BK == 32;
  constexpr int P = SWZ ? BK : BK + 8;           // LDS row pitch (elements)
  constexpr int A_ELEMS = BM * P;
  constexpr int B_ELEMS = BN * P;
  constexpr int STAGE = A_ELEMS + B_ELEMS;
  constexpr int CPR_A = BK / 8;                  // 16-byte chunks per A (and bf16 B) row
  constexpr int RPP_A = 256 / CPR_A;             // rows per load pass
  constexpr int A_CH = BM / RPP_A;               // 16-byte A chunks per thread
  constexpr int CPR_B = INT8B ? BK / 16 : BK / 8;
  constexpr int RPP_B = 256 / CPR_B;
  constexpr int B_CH = (BN + RPP_B - 1) / RPP_B;  // threads past row BN-1 hold no B chunk
  constexpr int WAVES_N = 4 / WAVES_M;
  constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;  // wave tile
  constexpr int MB = WM / 32, NB = WN / 32;            // MFMA blocks per wave
  static_assert(MB >= 1 && NB >= 1 && A_CH >= 1 && B_CH >= 1, "tile too small");
  static_assert(PF == 1 || PF == 2, "prefetch depth");
  constexpr int CP = BN + 8;  // C tile pitch in LDS (elements), epilogue
  constexpr int SMEM = 2 * STAGE > BM * CP ? 2 * STAGE : BM * CP;
  __shared__ __attribute__((aligned(16))) bf16 smem[SMEM];
  // element offset of 16-byte chunk `chunk` within LDS row `row`
  auto chunk_at = [](int row, int chunk) { return (SWZ ? chunk ^ ((row >> 2) & 3) : chunk) * 8; };

  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6, g = lane >> 5, c = lane & 31;
  const int wm = w / WAVES_N, wn = w % WAVES_N;

  const int tiles_m = (p.M + BM - 1) / BM;
  const int tiles_n = (p.N + BN - 1) / BN;
  const int n_tiles = tiles_m * tiles_n;
  const int id = xcd_remap(blockIdx.x, gridDim.x);
  const int tile = id % n_tiles;
  const int split = id / n_tiles;  // 0 unless split-K
  // Consecutive tiles (one XCD's run) share an operand through its L2
  // (p.n_fast: the larger operand, chosen on the host).
  const bool n_fast = p.n_fast != 0;
  const int tm = n_fast ? tile / tiles_n : tile % tiles_m;
  const int tn = n_fast ? tile % tiles_n : tile / tiles_m;
  const int m0 = tm * BM, n0 = tn * BN;
  const int n_k_all = (p.K + BK - 1) / BK;
  const int kt_begin = p.ws != nullptr ? split * p.kt_split : 0;
  const int kt_end = p.ws != nullptr ? min(n_k_all, kt_begin + p.kt_split) : n_k_all;
  const int k_first = kt_begin * BK;

  // ── per-thread A row state ────────────────────────────────────────────
  // The vector paths load through buffer resources, unconditionally: a
  // chunk that must read as zero (k past K, a padding tap of the conv
  // gather) gets the offset kOffNone, and rows past M (past N for B) read
  // the last valid row, whose products only reach discarded outputs.  No
  // branches, no zeroing moves, exact vmcnt counts for the compiler.
  const int a_col = (tid % CPR_A) * 8;  // k offset of this thread's chunk inside the tile
  const __amdgpu_buffer_rsrc_t a_rsrc = buffer_rsrc(p.A, p.a_bytes);
  const __amdgpu_buffer_rsrc_t b_rsrc = buffer_rsrc(p.B, p.b_bytes);
  int a_row[A_CH];
  bool a_ok[A_CH];
  const bf16 *a_base[A_CH];  // element paths: plain row / the row's image
  int a_ih0[A_CH], a_iw0[A_CH];
  int a_off[A_CH];  // vector paths, bytes: plain row start / conv tap (0, 0), channel 0
#pragma unroll
  for (int i = 0; i < A_CH; ++i) {
    a_row[i] = tid / CPR_A + RPP_A * i;
    const int m = m0 + a_row[i];
    a_ok[i] = m < p.M;
    const int mm = a_ok[i] ? m : p.M - 1;
    if constexpr (AMODE == kAPlain) {
      a_base[i] = p.A + static_cast<int64_t>(mm) * p.lda;
      a_ih0[i] = a_iw0[i] = 0;
      a_off[i] = static_cast<int>(static_cast<int64_t>(mm) * p.lda * 2);
    } else {
      const int ow = mm % p.OW;
      const int t = mm / p.OW;
      const int oh = t % p.OH;
      const int b = t / p.OH;
      a_ih0[i] = oh * p.SH - p.PH;
      a_iw0[i] = ow * p.SW - p.PW;
      const int64_t img = static_cast<int64_t>(b) * p.H * p.W * cst;
      a_base[i] = p.A + img;
      a_off[i] = static_cast<int>(2 * (img + static_cast<int64_t>(a_ih0[i] * p.W + a_iw0[i]) * cst));
    }
  }
  // Implicit-GEMM k decomposition (vector mode), stepped per k-tile: tap
  // (kh, kw), channel ci and the byte offset 2 ((kh W + kw) C_IN + ci).  When
  // C_IN is a multiple of BK a k-tile never straddles a tap, so the state of
  // the tile's first column is wave-uniform (scalar registers, scalar
  // branches) and a thread adds its column a_col; otherwise each thread
  // steps its own column.
  const bool tap_uniform = AMODE == kAConvVec && p.Cin % BK == 0;
  struct TapState {
    int ci, kw, kh, off;
  };
  auto tap_at = [&](int k) {
    TapState t;
    t.ci = k % p.Cin;
    const int r = k / p.Cin;
    t.kw = r % p.KW;
    t.kh = r / p.KW;
    t.off = 2 * ((t.kh * p.W + t.kw) * cst + t.ci);
    return t;
  };
  // u: the k-tile's first column (uniform); v: this thread's column
  TapState u_tap{0, 0, 0, 0}, v_tap{0, 0, 0, 0};
  if constexpr (AMODE == kAConvVec) {
    if (tap_uniform) u_tap = tap_at(k_first);
    else v_tap = tap_at(k_first + a_col);
  }
  // advance by one k-tile: the offset moves by BK elements, plus
  // cst - C_IN each time kw steps and (W - KW) cst each time kh steps
  auto tap_step = [&](TapState &t, bool once) __attribute__((always_inline)) {
    t.ci += BK;
    t.off += 2 * BK;
    while (t.ci >= p.Cin) {
      t.ci -= p.Cin;
      t.off += 2 * (cst - p.Cin);
      if (++t.kw == p.KW) {
        t.kw = 0;
        ++t.kh;
        t.off += 2 * (p.W - p.KW) * cst;
      }
      if (once) break;  // uniform case: C_IN % BK == 0, at most one step
    }
  };

  auto load_a = [&](int k0, u32x4 (&areg)[A_CH]) __attribute__((always_inline)) {
    const int k = k0 + a_col;
#pragma unroll
    for (int i = 0; i < A_CH; ++i) {
      if constexpr (AMODE == kAPlain && KVEC) {
        areg[i] = buffer_load16(a_rsrc, k < p.K ? a_off[i] + 2 * k : kOffNone);
      } else if constexpr (AMODE == kAPlain) {
        u32x4 v = u32x4{0u, 0u, 0u, 0u};
        if (a_ok[i] && k + 8 <= p.K) {
          v = *reinterpret_cast<const u32x4 *>(a_base[i] + k);
        } else if (a_ok[i] && k < p.K) {
          bf16 e[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) e[j] = k + j < p.K ? a_base[i][k + j] : static_cast<bf16>(0.0f);
          __builtin_memcpy(&v, e, 16);
        }
        areg[i] = v;
      } else if constexpr (AMODE == kAConvVec) {
        // (non-short-circuit: no branch)
        auto gather = [&](const TapState &t, int col_bytes) __attribute__((always_inline)) {
          const int ih = a_ih0[i] + t.kh, iw = a_iw0[i] + t.kw;
          const bool ok = (k < p.K) & (static_cast<unsigned>(ih) < static_cast<unsigned>(p.H)) &
                          (static_cast<unsigned>(iw) < static_cast<unsigned>(p.W));
          return buffer_load16(a_rsrc, ok ? a_off[i] + t.off + col_bytes : kOffNone);
        };
        areg[i] = tap_uniform ? gather(u_tap, 2 * a_col) : gather(v_tap, 0);
      } else {
        // element-wise gather (C_IN % 8 != 0, e.g. the 3-channel stem): the
        // chunk's first (ci, kw, kh) is decoded once, then stepped
        u32x4 v;
        bf16 e[8];
        int ci = k % p.Cin;
        const int r = k / p.Cin;
        int kw = r % p.KW, kh = r / p.KW;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          e[j] = static_cast<bf16>(0.0f);
          const int ih = a_ih0[i] + kh, iw = a_iw0[i] + kw;
          if (a_ok[i] && k + j < p.K && ih >= 0 && ih < p.H && iw >= 0 && iw < p.W)
            e[j] = a_base[i][(static_cast<int64_t>(ih) * p.W + iw) * cst + ci];
          if (++ci == p.Cin) {
            ci = 0;
            if (++kw == p.KW) {
              kw = 0;
              ++kh;
            }
          }
        }
        __builtin_memcpy(&v, e, 16);
        areg[i] = v;
      }
    }
    if constexpr (AMODE == kAConvVec) {
      if (tap_uniform) tap_step(u_tap, true);
      else tap_step(v_tap, false);
    }
  };

  // B rows (clamped into [0, N)), resolved once; a k-tile adds its k offset
  constexpr int B_ES = INT8B ? 1 : 2;  // bytes per B element
  int b_off[B_CH];
  const char *b_row_ptr[B_CH];
#pragma unroll
  for (int i = 0; i < B_CH; ++i) {
    const int row = tid / CPR_B + RPP_B * i;
    const int n = min(n0 + row, p.N - 1);
    b_off[i] = static_cast<int>(static_cast<int64_t>(n) * p.ldb * B_ES);
    b_row_ptr[i] = static_cast<const char *>(p.B) + static_cast<int64_t>(n) * p.ldb * B_ES;
  }
  auto load_b = [&](int k0, u32x4 (&breg)[B_CH]) __attribute__((always_inline)) {
    const int k = k0 + (tid % CPR_B) * (16 / B_ES);
#pragma unroll
    for (int i = 0; i < B_CH; ++i) {
      const int row = tid / CPR_B + RPP_B * i;
      if (RPP_B * (i + 1) > BN && row >= BN) {  // only when BN is not a whole number of passes
        breg[i] = u32x4{0u, 0u, 0u, 0u};
        continue;
      }
      if (INT8B || (KVEC && AMODE != kAConvScalar)) {
        breg[i] = buffer_load16(b_rsrc, k < p.K ? b_off[i] + B_ES * k : kOffNone);
      } else {
        // element-wise when rows are not 16-byte aligned (scalar-gather conv,
        // where ldb = KH*KW*C_IN is arbitrary) or the chunk straddles K
        const int n = n0 + row;
        const bf16 *brow = reinterpret_cast<const bf16 *>(b_row_ptr[i]);
        u32x4 v = u32x4{0u, 0u, 0u, 0u};
        if (AMODE != kAConvScalar && n < p.N && k + 8 <= p.K) {
          v = *reinterpret_cast<const u32x4 *>(brow + k);
        } else if (n < p.N && k < p.K) {
          bf16 e[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) e[j] = k + j < p.K ? brow[k + j] : static_cast<bf16>(0.0f);
          __builtin_memcpy(&v, e, 16);
        }
        breg[i] = v;
      }
    }
  };

  auto store_stage = [&](int buf, const u32x4 (&areg)[A_CH], const u32x4 (&breg)[B_CH]) __attribute__((always_inline)) {
    bf16 *as = smem + buf * STAGE;
    bf16 *bs = as + A_ELEMS;
#pragma unroll
    for (int i = 0; i < A_CH; ++i)
      *reinterpret_cast<u32x4 *>(as + a_row[i] * P + chunk_at(a_row[i], tid % CPR_A)) = areg[i];
#pragma unroll
    for (int i = 0; i < B_CH; ++i) {
      const int row = tid / CPR_B + RPP_B * i;
      if (RPP_B * (i + 1) > BN && row >= BN) continue;
      if constexpr (INT8B) {
        const int col = (tid % CPR_B) * 16;
        bf16 e[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int8_t q = static_cast<int8_t>((breg[i][j >> 2] >> (8 * (j & 3))) & 0xffu);
          e[j] = static_cast<bf16>(static_cast<float>(q));
        }
        u32x4 lo, hi;
        __builtin_memcpy(&lo, e, 16);
        __builtin_memcpy(&hi, e + 8, 16);
        *reinterpret_cast<u32x4 *>(bs + row * P + chunk_at(row, col / 8)) = lo;
        *reinterpret_cast<u32x4 *>(bs + row * P + chunk_at(row, col / 8 + 1)) = hi;
      } else {
        *reinterpret_cast<u32x4 *>(bs + row * P + chunk_at(row, tid % CPR_B)) = breg[i];
      }
    }
  };

  f32x16 acc[NB][MB];
#pragma unroll
  for (int i = 0; i < NB; ++i)
#pragma unroll
    for (int j = 0; j < MB; ++j) acc[i][j] = zero16();

  // Fragments of k-step s+1 are read before the MFMAs of step s issue; the
  // two fragment sets are separate variables (no runtime-indexed arrays).
  auto compute = [&](int stage) __attribute__((always_inline)) {
    const bf16 *as = smem + stage * STAGE;
    const bf16 *bs = as + A_ELEMS;
    bf16x8 w0[NB], x0[MB], w1[NB], x1[MB];
    auto read_frags = [&](int s, bf16x8 (&wf)[NB], bf16x8 (&xf)[MB]) __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < NB; ++i)
        wf[i] = *reinterpret_cast<const bf16x8 *>(bs + (wn * WN + i * 32 + c) * P + chunk_at(c, 2 * s + g));
#pragma unroll
      for (int j = 0; j < MB; ++j)
        xf[j] = *reinterpret_cast<const bf16x8 *>(as + (wm * WM + j * 32 + c) * P + chunk_at(c, 2 * s + g));
    };
    auto mma = [&](const bf16x8 (&wf)[NB], const bf16x8 (&xf)[MB]) __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < NB; ++i)
#pragma unroll
        for (int j = 0; j < MB; ++j) acc[i][j] = mfma32x32x16(wf[i], xf[j], acc[i][j]);
    };
    constexpr int S = BK / 16;
    static_assert(S % 2 == 0, "BK must be a multiple of 32");
    read_frags(0, w0, x0);
#pragma unroll
    for (int s = 0; s < S; s += 2) {
      read_frags(s + 1, w1, x1);
      mma(w0, x0);
      if (s + 2 < S) read_frags(s + 2, w0, x0);
      mma(w1, x1);
    }
  };

  // k-tiles of this workgroup (all of K unless split-K): kt counts from 0
  // and k offsets are k_first + kt * BK
  const int n_k = kt_end - kt_begin;
  if constexpr (PF == 1) {
    // one register set: tile kt+1 is fetched while tile kt is multiplied
    u32x4 ra[A_CH], rb[B_CH];
    load_a(k_first, ra);
    load_b(k_first, rb);
    store_stage(0, ra, rb);
    __syncthreads();
    for (int kt = 0; kt < n_k; ++kt) {
      if (kt + 1 < n_k) {
        load_a(k_first + (kt + 1) * BK, ra);
        load_b(k_first + (kt + 1) * BK, rb);
      }
      compute(kt & 1);
      if (kt + 1 < n_k) store_stage((kt + 1) & 1, ra, rb);
      __syncthreads();
    }
  } else {
    // two register sets (loop unrolled by two so the sets are named
    // statically): a tile's loads have two k-tiles of MFMA work to land.
    // With the buffer-load paths the loads are issued unconditionally: past
    // the last k-tile they are given k = K, which puts every lane's offset
    // out of range (zeros, no memory access).  A branch around the loads
    // would make the compiler's wait before the LDS stores assume the path
    // without them and drain the set just issued too (depth 1, not 2).
    constexpr bool kDeadLoads = AMODE == kAConvVec || (AMODE == kAPlain && KVEC);
    u32x4 ra0[A_CH], rb0[B_CH], ra1[A_CH], rb1[B_CH];
    load_a(k_first, ra0);
    load_b(k_first, rb0);
    if (kDeadLoads || n_k > 1) {
      const int k1 = n_k > 1 ? k_first + BK : p.K;
      load_a(k1, ra1);
      load_b(k1, rb1);
    }
    store_stage(0, ra0, rb0);
    __syncthreads();
    // next_*: the set holding tile kt+1; free_*: the set tile kt+2 is loaded into
    auto step = [&](int kt, const u32x4 (&next_a)[A_CH], const u32x4 (&next_b)[B_CH],
                    u32x4 (&free_a)[A_CH], u32x4 (&free_b)[B_CH]) __attribute__((always_inline)) {
      if (kDeadLoads || kt + 2 < n_k) {
        const int k2 = kt + 2 < n_k ? k_first + (kt + 2) * BK : p.K;
        load_a(k2, free_a);
        load_b(k2, free_b);
      }
      if (!kDeadLoads || kt < n_k) {
        compute(kt & 1);
        if (kt + 1 < n_k) store_stage((kt + 1) & 1, next_a, next_b);
        __syncthreads();
      }
    };
    for (int kt = 0; kt < n_k; kt += 2) {
      step(kt, ra1, rb1, ra0, rb0);
      if (kDeadLoads || kt + 1 < n_k) step(kt + 1, ra0, rb0, ra1, rb1);
    }
  }

  // ── epilogue ───────────────────────────────────────────────────────────
  // scale / bias / activation on the fp32 accumulators, bf16 tile staged in
  // LDS (the k-loop's last barrier freed it), then written back as 16-byte
  // row chunks: fully coalesced, unlike the accumulator layout (4 consecutive
  // n per lane, rows spread over lanes).  Loops are fully unrolled so every
  // accumulator index is static and the accumulators stay in registers.
  if (p.ws != nullptr) {
    // split-K partial: raw fp32 accumulators, four consecutive n per lane
    // (16-byte stores; the four v4 stores of a lane cover 128 contiguous
    // bytes of the row between the two lane halves)
    float *wsp = p.ws + static_cast<int64_t>(split) * p.M * p.N;
#pragma clang loop unroll(full)
    for (int j = 0; j < MB; ++j) {
      const int m = m0 + wm * WM + j * 32 + c;
#pragma clang loop unroll(full)
      for (int i = 0; i < NB; ++i) {
#pragma clang loop unroll(full)
        for (int v4 = 0; v4 < 4; ++v4) {
          const int n = n0 + wn * WN + i * 32 + 8 * v4 + 4 * g;
          if (m < p.M && n < p.N) {
            float *dst = wsp + static_cast<int64_t>(m) * p.N + n;
            if (n + 4 <= p.N && (p.N & 3) == 0) {
              f32x4 v{acc[i][j][4 * v4], acc[i][j][4 * v4 + 1], acc[i][j][4 * v4 + 2], acc[i][j][4 * v4 + 3]};
              *reinterpret_cast<f32x4 *>(dst) = v;
            } else {
              for (int e = 0; e < 4 && n + e < p.N; ++e) dst[e] = acc[i][j][4 * v4 + e];
            }
          }
        }
      }
    }
    return;
  }
  static_assert(WN % 16 == 0 && WM % 16 == 0, "fragment rows keep the swizzle of lane c");
  bf16 *cs = smem;
  // scale / bias per group of four columns (shared by the MB row blocks)
#pragma clang loop unroll(full)
  for (int i = 0; i < NB; ++i)
#pragma clang loop unroll(full)
    for (int v4 = 0; v4 < 4; ++v4) {
      float mul[4], add[4];
      epi_coeffs(p, n0 + wn * WN + i * 32 + 8 * v4 + 4 * g, mul, add);
#pragma clang loop unroll(full)
      for (int j = 0; j < MB; ++j)
#pragma clang loop unroll(full)
        for (int e = 0; e < 4; ++e) acc[i][j][4 * v4 + e] = __builtin_fmaf(acc[i][j][4 * v4 + e], mul[e], add[e]);
    }
  const EpiAct ea = epi_act(p.act);
  if (ea.sig) {
#pragma clang loop unroll(full)
    for (int i = 0; i < NB; ++i)
#pragma clang loop unroll(full)
      for (int j = 0; j < MB; ++j)
#pragma clang loop unroll(full)
        for (int v = 0; v < 16; ++v) acc[i][j][v] = epi_sig(acc[i][j][v], ea);
  }
  const float lo = ea.relu ? 0.0f : -INFINITY;
#pragma clang loop unroll(full)
  for (int j = 0; j < MB; ++j) {
    const int ml = wm * WM + j * 32 + c;
#pragma clang loop unroll(full)
    for (int i = 0; i < NB; ++i) {
#pragma clang loop unroll(full)
      for (int v4 = 0; v4 < 4; ++v4) {
        const int nl = wn * WN + i * 32 + 8 * v4 + 4 * g;
        bf16x4 o4;
#pragma clang loop unroll(full)
        for (int e = 0; e < 4; ++e) {
          const float r = acc[i][j][4 * v4 + e];
          o4[e] = static_cast<bf16>(r < lo ? lo : r);
        }
        // 16-byte chunk nl / 8 of row ml sits at chunk (nl / 8) ^ ((ml >> 4) & 1):
        // rows c and c + 16 of one write instruction then use different banks
        *reinterpret_cast<bf16x4 *>(cs + ml * CP + (((nl >> 3) ^ ((ml >> 4) & 1)) << 3) + (nl & 7)) = o4;
      }
    }
  }
  __syncthreads();
  constexpr int CPR_C = BN / 8;        // 16-byte chunks per C row
  constexpr int RPP_C = 256 / CPR_C;   // rows per pass
  const bool vec16 = c_rows_vec16(p);
#pragma clang loop unroll(full)
  for (int r0 = 0; r0 < BM; r0 += RPP_C) {
    const int ml = r0 + tid / CPR_C, nl = (tid % CPR_C) * 8;
    const int m = m0 + ml, n = n0 + nl;
    if (m < p.M && n < p.N) {
      const u32x4 v = *reinterpret_cast<const u32x4 *>(cs + ml * CP + (((nl >> 3) ^ ((ml >> 4) & 1)) << 3));
      bf16 *dst = p.C + c_row(p, m) + n;
      if (vec16 && n + 8 <= p.N) {
        *reinterpret_cast<u32x4 *>(dst) = v;
      } else {
        bf16 e[8];
        __builtin_memcpy(e, &v, 16);
        for (int t = 0; t < 8 && n + t < p.N; ++t) dst[t] = e[t];
      }
    }
  }
}

// Sums the split-K partials ws[0..S)[m][n] and applies scale / bias /
// activation; eight consecutive n per thread (16-byte bf16 stores).
static __global__ __launch_bounds__(256) void gemm_splitk_finalize(GemmParams p, int S) {
  const int64_t groups_per_row = (p.N + 7) / 8;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (gid >= groups_per_row * p.M) return;
  const int m = static_cast<int>(gid / groups_per_row);
  const int n0 = static_cast<int>(gid % groups_per_row) * 8;
  const int64_t plane = static_cast<int64_t>(p.M) * p.N;
  const float *src = p.ws + static_cast<int64_t>(m) * p.N + n0;
  float r[8];
  const bool vec = (p.N & 7) == 0;
  if (vec) {
    f32x4 a = *reinterpret_cast<const f32x4 *>(src), b = *reinterpret_cast<const f32x4 *>(src + 4);
    for (int sp = 1; sp < S; ++sp) {
      a += *reinterpret_cast<const f32x4 *>(src + sp * plane);
      b += *reinterpret_cast<const f32x4 *>(src + sp * plane + 4);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      r[e] = a[e];
      r[e + 4] = b[e];
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      r[e] = 0.0f;
      if (n0 + e < p.N)
        for (int sp = 0; sp < S; ++sp) r[e] += src[sp * plane + e];
    }
  }
  bf16 o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int n = n0 + e;
    float v = r[e];
    if (n < p.N) {
      if (p.scale != nullptr) v *= p.scale[n];
      if (p.bias != nullptr) v += p.bias[n];
      if (p.bias_bf16 != nullptr) v += static_cast<float>(p.bias_bf16[n]);
    }
    o[e] = static_cast<bf16>(apply_act_rt(v, p.act));
  }
  bf16 *dst = p.C + c_row(p, m) + n0;
  if (vec && c_rows_vec16(p)) {
    u32x4 v;
    __builtin_memcpy(&v, o, 16);
    *reinterpret_cast<u32x4 *>(dst) = v;
  } else {
    for (int e = 0; e < 8 && n0 + e < p.N; ++e) dst[e] = o[e];
  }
}


// KVEC: K % 8 == 0 and (for the plain A path) 16-byte aligned rows, so no
// 16-byte chunk straddles K and the element-wise tail paths are compiled out.
template <int BM, int BN, int BK, int WAVES_M, int PF, bool INT8B, int AMODE>
inline void launch_tile(const GemmParams &p, hipStream_t s, int splits = 1) {
  const int grid = ((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN) * splits;
  const unsigned groups = p.groups > 1 ? static_cast<unsigned>(p.groups) : 1u;
  if (p.K % 8 == 0 && AMODE != kAConvScalar) {
    hipLaunchKernelGGL((gemm_mfma_kernel<BM, BN, BK, WAVES_M, PF, INT8B, AMODE, true>), dim3(grid, groups),
                       dim3(256), 0, s, p);
  } else {
    hipLaunchKernelGGL((gemm_mfma_kernel<BM, BN, BK, WAVES_M, PF, INT8B, AMODE, false>), dim3(grid, groups),
                       dim3(256), 0, s, p);
  }
}

inline int64_t tiles_of(const GemmParams &p, int bm, int bn) {
  return static_cast<int64_t>((p.M + bm - 1) / bm) * ((p.N + bn - 1) / bn);
}

// Host launcher: 128 x 128 x 64 tiles (two workgroups per CU); narrow
// outputs (N <= 64, e.g. the 64-channel convs) and grids that 128 x 128
// tiles leave short of the CU count take 128 x 64 x 32 tiles with a
// two-tile prefetch.  Measured on MI355X, larger tiles (256 x 128,
// 256 x 256 with AGPR accumulators and one workgroup per CU) were no faster
// for these shapes.
// Split-K factor for a BM x BN x BK tiling: only deep-K problems (K >= 2048)
// whose tiles cover fewer than half the CUs (ResNet stage 4: 100 tiles, K =
// 2048 and 4608) are split, towards two workgroups per CU, with at most
// four splits (the fp32 partials cost 8 * S * M * N bytes of extra
// traffic).  Measured on MI355X: at 196 tiles (stage 3) splitting does not
// pay; the 7x7 3x3 512 -> 512 layers (K = 4608) take 36 us with four
// splits against 44, 41, 43 and 44 us with 2, 3, 6 and 8.
inline int splitk_factor(const GemmParams &p, int bm, int bn, int bk) {
  const int64_t tiles = tiles_of(p, bm, bn);
  const int n_k = (p.K + bk - 1) / bk;
  const int64_t cus = device_cu_count();
  const int64_t target = 2 * cus;
  if (2 * tiles >= cus || n_k * bk < 2048) return 1;
  int sp = static_cast<int>((target + tiles - 1) / tiles);
  sp = min(sp, min(4, n_k / 4));
  return max(sp, 1);
}

// Split plan: how many K slices hold k-tiles and the bytes of their fp32
// partial sums (used == 1: no split).
struct SplitPlan {
  int used = 1;
  int kt_split = 0;
  size_t bytes = 0;
};

template <int BM, int BN, int BK>
inline SplitPlan split_plan(const GemmParams &p) {
  SplitPlan sp;
  const int f = splitk_factor(p, BM, BN, BK);
  if (f > 1) {
    const int n_k = (p.K + BK - 1) / BK;
    sp.kt_split = (n_k + f - 1) / f;
    sp.used = (n_k + sp.kt_split - 1) / sp.kt_split;
    sp.bytes = static_cast<size_t>(sp.used) * p.M * p.N * sizeof(float);
  }
  return sp;
}

// Runs split along K when the plan splits and the caller's scratch holds the
// partial sums; otherwise unsplit (same products, one accumulation chain).
template <int BM, int BN, int BK, int WAVES_M, int PF, bool INT8B, int AMODE>
inline void launch_split(GemmParams p, hipStream_t s, Scratch scr) {
  const SplitPlan sp = split_plan<BM, BN, BK>(p);
  if (sp.used > 1 && scr.ptr != nullptr && scr.bytes >= sp.bytes) {
    p.ws = static_cast<float *>(scr.ptr);
    p.kt_split = sp.kt_split;
    launch_tile<BM, BN, BK, WAVES_M, PF, INT8B, AMODE>(p, s, sp.used);
    const int64_t groups = static_cast<int64_t>(p.M) * ((p.N + 7) / 8);
    hipLaunchKernelGGL(gemm_splitk_finalize, dim3(static_cast<unsigned>((groups + 255) / 256)), dim3(256), 0,
                       s, p, sp.used);
    return;
  }
  p.ws = nullptr;
  launch_tile<BM, BN, BK, WAVES_M, PF, INT8B, AMODE>(p, s);
}

template <bool INT8B, int AMODE>
inline bool big_gemm_fits(const GemmParams &p);
template <bool INT8B, int AMODE>
inline void launch_big_gemm(GemmParams p, hipStream_t s);
template <bool INT8B, int AMODE>
inline bool stream_gemm_fits(const GemmParams &p);
inline void launch_stream_gemm(const GemmParams &p, hipStream_t s);
template <bool INT8B, int AMODE>
inline bool persist_gemm_fits(const GemmParams &p);
template <int AMODE>
inline void launch_persist_default(const GemmParams &p, hipStream_t s);

// Tile choice (measured on MI355X over the ResNet-50 and W8A16 shapes):
//  * the persistent LDS-DMA kernel (gemm_persist.hpp) for bf16 problems of
//    many 128 x 128 tiles (>= 1.5 per CU) and K of 128 .. 512, or up to 1024
//    for N <= 1024 (the 1x1 and strided 1x1 convs of a ResNet's second and
//    third stages);
//  * the streaming kernel (gemm_stream.hpp) for long, HBM-bound problems
//    with K, N <= 256 and bf16 weights (the full-resolution 1x1 convs);
//  * the 256 x 256 LDS-DMA kernel (gemm_dma.hpp) when its tiles fill the chip;
//  * narrow outputs (N <= 64): 64 x 64 x 64 tiles for deep K (more
//    workgroups to hide latency), else 128 x 64 x 32;
//  * short K (<= 256, the 1x1 convs): 128 x 128 x 32 with a two-tile
//    prefetch, so the few k-tiles still overlap loads with MFMAs;
//  * grids of 128 x 128 tiles that leave CUs idle and do not split along K:
//    128 x 64 x 64 (twice the workgroups);
//  * otherwise 128 x 128 x 64, split along K when badly under-filled (the
//    int8 3x3 conv 32 x 256 x 28 x 28 -> 256, 392 tiles: 48.7 us, against
//    54.4 us for 128 x 128 x 32 with the two-tile prefetch and 70 us for
//    128 x 64 x 64).
enum GemmTiles { kTilesPersist, kTilesStream, kTilesBig, kTiles128x64, kTiles64x64, kTiles128x128Short, kTiles128x64Deep, kTiles128x128 };

template <bool INT8B, int AMODE>
inline GemmTiles gemm_tiles(const GemmParams &p) {
  const bool plain_rows = p.c_ow <= 0;  // remapped rows: register-staged kernels only
  if (plain_rows && persist_gemm_fits<INT8B, AMODE>(p)) return kTilesPersist;
  if (plain_rows && stream_gemm_fits<INT8B, AMODE>(p)) return kTilesStream;
  if constexpr (AMODE != kAConvScalar) {
    if (plain_rows && big_gemm_fits<INT8B, AMODE>(p)) return kTilesBig;
  }
  if (p.N <= 64) return p.K >= 512 ? kTiles64x64 : kTiles128x64;
  if (p.K <= 256) return kTiles128x128Short;
  // 128 x 64 tiles with a two-tile prefetch when 128 x 128 tiles leave CUs
  // idle: unsplit up to K = 2048 (7x7 2048 -> 512: 17.5 us against 25 us
  // for four K slices plus their reduction), split beyond (a 4608-deep K
  // chain of 72 k-tiles is long enough that slicing it wins)
  if (tiles_of(p, 128, 128) < device_cu_count() && (split_plan<128, 128, 64>(p).used == 1 || p.K <= 2048))
    return kTiles128x64Deep;
  return kTiles128x128;
}

// Scratch bytes that let launch_gemm_mfma take its split plan (0: none used).
template <bool INT8B, int AMODE>
inline size_t gemm_scratch_bytes(const GemmParams &p) {
  switch (gemm_tiles<INT8B, AMODE>(p)) {
    case kTiles128x64: return split_plan<128, 64, 32>(p).bytes;
    case kTiles64x64: return split_plan<64, 64, 64>(p).bytes;
    case kTiles128x128Short: return split_plan<128, 128, 32>(p).bytes;
    case kTiles128x64Deep: return split_plan<128, 64, 64>(p).bytes;
    case kTiles128x128: return split_plan<128, 128, 64>(p).bytes;
    default: return 0;
  }
}

// Byte extents of the A and B operands as the kernels address them.
template <bool INT8B, int AMODE>
inline int64_t gemm_a_extent(const GemmParams &p) {
  if (AMODE == kAPlain) return (static_cast<int64_t>(p.M - 1) * p.lda + p.K) * 2;
  return static_cast<int64_t>(p.M / (p.OH * p.OW)) * p.H * p.W * p.Cin * 2;  // whole images
}
template <bool INT8B>
inline int64_t gemm_b_extent(const GemmParams &p) {
  return (static_cast<int64_t>(p.N - 1) * p.ldb + p.K) * (INT8B ? 1 : 2);
}

// Grouped conv on the register-staged kernels, all groups in one launch
// (workgroup row blockIdx.y = group; GemmParams::groups): no split along K.
// False (nothing launched) when an operand's extent reaches 2^31 bytes.
template <bool INT8B, int AMODE>
inline bool launch_grouped_gemm(GemmParams p, int act, hipStream_t s) {
  if (act < TEENY_ACT_NONE || act > TEENY_ACT_SILU || p.groups < 2) return false;
  constexpr int64_t kMaxExtent = 0x7fffffff;
  const int64_t a_ext = AMODE == kAPlain
                            ? (static_cast<int64_t>(p.M - 1) * p.lda + p.cst) * 2
                            : static_cast<int64_t>(p.M / (p.OH * p.OW)) * p.H * p.W * p.cst * 2;
  const int64_t b_ext = static_cast<int64_t>(p.groups) * p.g_b * (INT8B ? 1 : 2);
  if (a_ext > kMaxExtent || b_ext > kMaxExtent || static_cast<int64_t>(p.M) * p.ldc * 2 > kMaxExtent) return false;
  p.a_bytes = static_cast<int>(a_ext);
  p.b_bytes = static_cast<int>(b_ext);
  p.n_fast = static_cast<int64_t>(p.M) * p.K * 2 > static_cast<int64_t>(p.N) * p.K * (INT8B ? 1 : 2);
  p.act = act;
  p.ws = nullptr;
  p.c_ow = 0;
  if (p.N <= 64) launch_tile<128, 64, 32, 2, 2, INT8B, AMODE>(p, s);
  else if (p.K <= 256) launch_tile<128, 128, 32, 2, 2, INT8B, AMODE>(p, s);
  else launch_tile<128, 128, 64, 2, 1, INT8B, AMODE>(p, s);
  return true;
}

template <bool INT8B, int AMODE>
inline bool launch_gemm_mfma(GemmParams p, int act, hipStream_t s, Scratch scr) {
  if (act < TEENY_ACT_NONE || act > TEENY_ACT_SILU) return false;
  constexpr int64_t kMaxExtent = 0x7fffffff;
  // Operands past 2^31 bytes (32-bit buffer offsets): run the problem as
  // row chunks of A (whole images for a conv) or column chunks of B, each
  // within the limit; the outputs are disjoint.
  if (gemm_a_extent<INT8B, AMODE>(p) > kMaxExtent) {
    const int64_t unit = AMODE == kAPlain ? 1 : static_cast<int64_t>(p.OH) * p.OW;  // rows per unit
    const int64_t unit_bytes = AMODE == kAPlain ? p.lda * 2 : static_cast<int64_t>(p.H) * p.W * p.Cin * 2;
    const int64_t per = std::max<int64_t>(1, (kMaxExtent - 2 * static_cast<int64_t>(p.K)) / unit_bytes);
    for (int64_t u0 = 0; u0 * unit < p.M; u0 += per) {
      GemmParams q = p;
      const int64_t m0 = u0 * unit;
      q.M = static_cast<int>(std::min<int64_t>(p.M - m0, per * unit));
      q.A = p.A + u0 * (AMODE == kAPlain ? p.lda : static_cast<int64_t>(p.H) * p.W * p.Cin);
      q.C = p.C + (p.c_ow > 0 ? u0 * p.c_sb : m0 * p.ldc);
      launch_gemm_mfma<INT8B, AMODE>(q, act, s, scr);
    }
    return true;
  }
  if (gemm_b_extent<INT8B>(p) > kMaxExtent) {
    const int64_t row_bytes = p.ldb * (INT8B ? 1 : 2);
    const int64_t per = std::max<int64_t>(8, (kMaxExtent - row_bytes) / row_bytes / 8 * 8);
    for (int64_t n0 = 0; n0 < p.N; n0 += per) {
      GemmParams q = p;
      q.N = static_cast<int>(std::min<int64_t>(p.N - n0, per));
      q.B = static_cast<const char *>(p.B) + n0 * row_bytes;
      q.C = p.C + n0;
      if (p.scale != nullptr) q.scale = p.scale + n0;
      if (p.bias != nullptr) q.bias = p.bias + n0;
      if (p.bias_bf16 != nullptr) q.bias_bf16 = p.bias_bf16 + n0;
      launch_gemm_mfma<INT8B, AMODE>(q, act, s, scr);
    }
    return true;
  }
  p.a_bytes = static_cast<int>(gemm_a_extent<INT8B, AMODE>(p));
  p.b_bytes = static_cast<int>(gemm_b_extent<INT8B>(p));
  // Share the larger operand between neighbouring tiles: A as the tiles
  // read it (M x K bf16, the implicit-GEMM view for a conv) against B.
  p.n_fast = static_cast<int64_t>(p.M) * p.K * 2 > static_cast<int64_t>(p.N) * p.K * (INT8B ? 1 : 2);
  p.act = act;
  p.ws = nullptr;
  switch (gemm_tiles<INT8B, AMODE>(p)) {
    case kTilesPersist:
      if constexpr (AMODE != kAConvScalar) launch_persist_default<AMODE>(p, s);
      break;
    case kTilesStream: launch_stream_gemm(p, s); break;
    case kTilesBig:
      if constexpr (AMODE != kAConvScalar) launch_big_gemm<INT8B, AMODE>(p, s);
      break;
    case kTiles128x64: launch_split<128, 64, 32, 2, 2, INT8B, AMODE>(p, s, scr); break;
    case kTiles64x64: launch_split<64, 64, 64, 2, 2, INT8B, AMODE>(p, s, scr); break;
    case kTiles128x128Short: launch_split<128, 128, 32, 2, 2, INT8B, AMODE>(p, s, scr); break;
    case kTiles128x64Deep: launch_split<128, 64, 64, 2, 2, INT8B, AMODE>(p, s, scr); break;
    default: launch_split<128, 128, 64, 2, 1, INT8B, AMODE>(p, s, scr); break;
  }
  return true;
}

}  // namespace teeny

#include "gemm_dma.hpp"
#include "gemm_stream.hpp"
#include "gemm_persist.hpp"
