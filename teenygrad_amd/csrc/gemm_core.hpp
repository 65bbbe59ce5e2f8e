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
// Tiling: BM x BN x 64 per workgroup of 256 threads (4 waves as 2 x 2), each
// wave a (BM/2) x (BN/2) block of v_mfma_f32_32x32x16_bf16 tiles.  The MFMA
// computes C^T (weights as the A operand, activations as the B operand) so
// each lane's accumulator column is one output row m and four consecutive
// registers are four consecutive n: the epilogue writes 8-byte bf16x4
// stores.  LDS rows are padded to 72 elements (144 B), which makes the
// 16-byte fragment reads of 16 consecutive rows hit 16 disjoint bank
// quads.  Two LDS stages: the next k-tile is fetched into registers before
// the current one is consumed and written to the other stage afterwards, so
// one barrier per k-tile suffices.
#pragma once

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
  // implicit-GEMM conv geometry (NHWC)
  int H, W, Cin, OH, OW, KH, KW, SH, SW, PH, PW;
};

constexpr int kGemmBK = 64;
constexpr int kGemmPitch = kGemmBK + 8;  // elements

template <int BM, int BN, bool INT8B, int AMODE, int ACT>
__global__ __launch_bounds__(256, 2) void gemm_mfma_kernel(GemmParams p) {
  constexpr int BK = kGemmBK;
  constexpr int P = kGemmPitch;
  constexpr int A_ELEMS = BM * P;
  constexpr int B_ELEMS = BN * P;
  constexpr int STAGE = A_ELEMS + B_ELEMS;
  constexpr int A_CH = BM / 32;                  // 16-byte A chunks per thread
  constexpr int B_CH = INT8B ? BN / 64 : BN / 32; // 16-byte B chunks per thread
  constexpr int WM = BM / 2, WN = BN / 2;        // wave tile
  constexpr int MB = WM / 32, NB = WN / 32;      // MFMA blocks per wave
  __shared__ __attribute__((aligned(16))) bf16 smem[2 * STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6, g = lane >> 5, c = lane & 31;
  const int wm = w >> 1, wn = w & 1;

  // Tile order: consecutive workgroups walk down M within a BN column so that
  // the B (weight) tile is shared through L2 by neighbours.
  const int tiles_m = (p.M + BM - 1) / BM;
  const int tm = blockIdx.x % tiles_m;
  const int tn = blockIdx.x / tiles_m;
  const int m0 = tm * BM, n0 = tn * BN;

  // ── per-thread A row state ────────────────────────────────────────────
  const int a_col = (tid & 7) * 8;  // k offset of this thread's chunk inside the tile
  int a_row[A_CH];
  bool a_ok[A_CH];
  const bf16 *a_base[A_CH];
  int a_ih0[A_CH], a_iw0[A_CH];
#pragma unroll
  for (int i = 0; i < A_CH; ++i) {
    a_row[i] = (tid >> 3) + 32 * i;
    const int m = m0 + a_row[i];
    a_ok[i] = m < p.M;
    if constexpr (AMODE == kAPlain) {
      a_base[i] = p.A + static_cast<int64_t>(a_ok[i] ? m : 0) * p.lda;
      a_ih0[i] = a_iw0[i] = 0;
    } else {
      const int mm = a_ok[i] ? m : 0;
      const int ow = mm % p.OW;
      const int t = mm / p.OW;
      const int oh = t % p.OH;
      const int b = t / p.OH;
      a_ih0[i] = oh * p.SH - p.PH;
      a_iw0[i] = ow * p.SW - p.PW;
      a_base[i] = p.A + static_cast<int64_t>(b) * p.H * p.W * p.Cin;
    }
  }
  // implicit-GEMM k decomposition of this thread's chunk column (vector mode)
  int k_ci = 0, k_kw = 0, k_kh = 0;
  if constexpr (AMODE == kAConvVec) {
    k_ci = a_col % p.Cin;
    const int r = a_col / p.Cin;
    k_kw = r % p.KW;
    k_kh = r / p.KW;
  }

  u32x4 areg[A_CH];
  u32x4 breg[B_CH];

  auto load_a = [&](int k0) {
#pragma unroll
    for (int i = 0; i < A_CH; ++i) {
      const int k = k0 + a_col;
      u32x4 v = u32x4{0u, 0u, 0u, 0u};
      if constexpr (AMODE == kAPlain) {
        if (a_ok[i] && k + 8 <= p.K) {
          v = *reinterpret_cast<const u32x4 *>(a_base[i] + k);
        } else if (a_ok[i] && k < p.K) {
          bf16 e[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) e[j] = k + j < p.K ? a_base[i][k + j] : static_cast<bf16>(0.0f);
          __builtin_memcpy(&v, e, 16);
        }
      } else if constexpr (AMODE == kAConvVec) {
        const int ih = a_ih0[i] + k_kh, iw = a_iw0[i] + k_kw;
        if (a_ok[i] && k < p.K && ih >= 0 && ih < p.H && iw >= 0 && iw < p.W)
          v = *reinterpret_cast<const u32x4 *>(a_base[i] + (static_cast<int64_t>(ih) * p.W + iw) * p.Cin + k_ci);
      } else {
        bf16 e[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int kk = k + j;
          e[j] = static_cast<bf16>(0.0f);
          if (a_ok[i] && kk < p.K) {
            const int ci = kk % p.Cin;
            const int r = kk / p.Cin;
            const int kw = r % p.KW, kh = r / p.KW;
            const int ih = a_ih0[i] + kh, iw = a_iw0[i] + kw;
            if (ih >= 0 && ih < p.H && iw >= 0 && iw < p.W)
              e[j] = a_base[i][(static_cast<int64_t>(ih) * p.W + iw) * p.Cin + ci];
          }
        }
        __builtin_memcpy(&v, e, 16);
      }
      areg[i] = v;
    }
    if constexpr (AMODE == kAConvVec) {
      // advance this thread's (kh, kw, ci) by one k-tile
      k_ci += BK;
      while (k_ci >= p.Cin) {
        k_ci -= p.Cin;
        if (++k_kw == p.KW) {
          k_kw = 0;
          ++k_kh;
        }
      }
    }
  };

  auto load_b = [&](int k0) {
#pragma unroll
    for (int i = 0; i < B_CH; ++i) {
      u32x4 v = u32x4{0u, 0u, 0u, 0u};
      if constexpr (INT8B) {
        const int row = (tid >> 2) + 64 * i;
        const int k = k0 + (tid & 3) * 16;
        const int n = n0 + row;
        if (n < p.N && k < p.K)
          v = *reinterpret_cast<const u32x4 *>(static_cast<const int8_t *>(p.B) + static_cast<int64_t>(n) * p.ldb + k);
      } else {
        const int row = (tid >> 3) + 32 * i;
        const int k = k0 + (tid & 7) * 8;
        const int n = n0 + row;
        const bf16 *brow = static_cast<const bf16 *>(p.B) + static_cast<int64_t>(n) * p.ldb;
        // Element-wise when rows are not 16-byte aligned (scalar-gather conv,
        // where ldb = KH*KW*C_IN is arbitrary) or the chunk straddles K.
        if (AMODE != kAConvScalar && n < p.N && k + 8 <= p.K) {
          v = *reinterpret_cast<const u32x4 *>(brow + k);
        } else if (n < p.N && k < p.K) {
          bf16 e[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) e[j] = k + j < p.K ? brow[k + j] : static_cast<bf16>(0.0f);
          __builtin_memcpy(&v, e, 16);
        }
      }
      breg[i] = v;
    }
  };

  auto store_stage = [&](int buf) {
    bf16 *as = smem + buf * STAGE;
    bf16 *bs = as + A_ELEMS;
#pragma unroll
    for (int i = 0; i < A_CH; ++i) *reinterpret_cast<u32x4 *>(as + a_row[i] * P + a_col) = areg[i];
#pragma unroll
    for (int i = 0; i < B_CH; ++i) {
      if constexpr (INT8B) {
        const int row = (tid >> 2) + 64 * i;
        const int col = (tid & 3) * 16;
        bf16 e[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int8_t q = static_cast<int8_t>((breg[i][j >> 2] >> (8 * (j & 3))) & 0xffu);
          e[j] = static_cast<bf16>(static_cast<float>(q));
        }
        u32x4 lo, hi;
        __builtin_memcpy(&lo, e, 16);
        __builtin_memcpy(&hi, e + 8, 16);
        *reinterpret_cast<u32x4 *>(bs + row * P + col) = lo;
        *reinterpret_cast<u32x4 *>(bs + row * P + col + 8) = hi;
      } else {
        const int row = (tid >> 3) + 32 * i;
        *reinterpret_cast<u32x4 *>(bs + row * P + (tid & 7) * 8) = breg[i];
      }
    }
  };

  f32x16 acc[NB][MB];
#pragma unroll
  for (int i = 0; i < NB; ++i)
#pragma unroll
    for (int j = 0; j < MB; ++j) acc[i][j] = zero16();

  const int n_k = (p.K + BK - 1) / BK;
  load_a(0);
  load_b(0);
  store_stage(0);
  __syncthreads();

  for (int kt = 0; kt < n_k; ++kt) {
    if (kt + 1 < n_k) {
      load_a((kt + 1) * BK);
      load_b((kt + 1) * BK);
    }
    const bf16 *as = smem + (kt & 1) * STAGE;
    const bf16 *bs = as + A_ELEMS;
#pragma unroll
    for (int s = 0; s < BK / 16; ++s) {
      bf16x8 wf[NB], xf[MB];
#pragma unroll
      for (int i = 0; i < NB; ++i)
        wf[i] = *reinterpret_cast<const bf16x8 *>(bs + (wn * WN + i * 32 + c) * P + 16 * s + 8 * g);
#pragma unroll
      for (int j = 0; j < MB; ++j)
        xf[j] = *reinterpret_cast<const bf16x8 *>(as + (wm * WM + j * 32 + c) * P + 16 * s + 8 * g);
#pragma unroll
      for (int i = 0; i < NB; ++i)
#pragma unroll
        for (int j = 0; j < MB; ++j) acc[i][j] = mfma32x32x16(wf[i], xf[j], acc[i][j]);
    }
    if (kt + 1 < n_k) store_stage((kt + 1) & 1);
    __syncthreads();
  }

  // ── epilogue ───────────────────────────────────────────────────────────
  const bool vec_store = (p.ldc % 4 == 0) && ((reinterpret_cast<uintptr_t>(p.C) & 7) == 0);
#pragma unroll
  for (int j = 0; j < MB; ++j) {
    const int m = m0 + wm * WM + j * 32 + c;
    if (m >= p.M) continue;
    bf16 *crow = p.C + static_cast<int64_t>(m) * p.ldc;
#pragma unroll
    for (int i = 0; i < NB; ++i) {
#pragma unroll
      for (int v4 = 0; v4 < 4; ++v4) {
        const int nb = n0 + wn * WN + i * 32 + 8 * v4 + 4 * g;
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int n = nb + e;
          float r = acc[i][j][4 * v4 + e];
          if (n < p.N) {
            if (p.scale != nullptr) r *= p.scale[n];
            if (p.bias != nullptr) r += p.bias[n];
            if (p.bias_bf16 != nullptr) r += static_cast<float>(p.bias_bf16[n]);
          }
          o[e] = apply_act<ACT, true>(r);
        }
        if (vec_store && nb + 3 < p.N) {
          bf16x4 o4;
#pragma unroll
          for (int e = 0; e < 4; ++e) o4[e] = static_cast<bf16>(o[e]);
          *reinterpret_cast<bf16x4 *>(crow + nb) = o4;
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (nb + e < p.N) crow[nb + e] = static_cast<bf16>(o[e]);
        }
      }
    }
  }
}

// Host launcher: picks the tile shape for the problem and instantiates the kernel.
template <bool INT8B, int AMODE, int ACT>
inline void launch_gemm_mfma_act(const GemmParams &p, hipStream_t s) {
  // BN = 64 tiles for narrow outputs (e.g. the 64-channel convs), else 128.
  if (p.N <= 64) {
    constexpr int BM = 128, BN = 64;
    const int grid = ((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN);
    hipLaunchKernelGGL((gemm_mfma_kernel<BM, BN, INT8B, AMODE, ACT>), dim3(grid), dim3(256), 0, s, p);
  } else {
    constexpr int BM = 128, BN = 128;
    const int grid = ((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN);
    hipLaunchKernelGGL((gemm_mfma_kernel<BM, BN, INT8B, AMODE, ACT>), dim3(grid), dim3(256), 0, s, p);
  }
}

template <bool INT8B, int AMODE>
inline bool launch_gemm_mfma(const GemmParams &p, int act, hipStream_t s) {
  switch (act) {
    case TEENY_ACT_NONE: launch_gemm_mfma_act<INT8B, AMODE, TEENY_ACT_NONE>(p, s); return true;
    case TEENY_ACT_RELU: launch_gemm_mfma_act<INT8B, AMODE, TEENY_ACT_RELU>(p, s); return true;
    case TEENY_ACT_GELU_TANH: launch_gemm_mfma_act<INT8B, AMODE, TEENY_ACT_GELU_TANH>(p, s); return true;
    case TEENY_ACT_SILU: launch_gemm_mfma_act<INT8B, AMODE, TEENY_ACT_SILU>(p, s); return true;
    default: return false;
  }
}

}  // namespace teeny
