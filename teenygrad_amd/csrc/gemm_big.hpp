// Large-tile MFMA GEMM for problems that fill the chip with 256 x 256 tiles
// (the W8A16 linears, big implicit-GEMM convs).  Same contract as
// gemm_mfma_kernel (gemm_core.hpp):
//
//   C[m, n] = act( scale[n] * sum_k A[m, k] * B[n, k] + bias[n] )
//
// with A bf16 (plain rows or the NHWC implicit-GEMM gather, C_IN % 8 == 0)
// and B bf16 or int8 [N][K].
//
// Why a second kernel: a 128 x 128 tile reads 1 KiB of LDS fragments per
// v_mfma_f32_32x32x16_bf16 (four waves, 64 x 64 each), which is the LDS
// bandwidth of a CU at the MFMA rate, so that kernel saturates LDS well
// before the matrix cores.  Here one workgroup of four waves owns a
// 256 x 256 tile and each wave a 128 x 128 block (16 MFMAs per k-step from
// 8 fragments: 0.5 KiB per MFMA).  Its accumulators (256 per lane) live in
// AGPRs, so there is one wave per SIMD and latency is hidden inside the
// wave instead of across waves:
//
//  * global -> LDS moves by LDS-DMA (global_load_lds_dwordx4, no staging
//    registers), issued from inline asm so the compiler neither counts it
//    nor waits on it before LDS reads of other stages; four LDS stages, the
//    DMA two k-tiles ahead, one barrier per k-tile (after an explicit
//    s_waitcnt vmcnt that leaves only this k-tile's DMA in flight).
//  * a k-tile is 32 fenced bundles, each one MFMA plus a share of the
//    other work: the DMA of k-tile kt+3, LDS reads that refill the one
//    fragment set in place 1..16 MFMAs ahead of use (k-tile kt+1's data is
//    complete and published once tile kt starts), and the int8 -> bf16
//    weight conversion.
//  * int8 weights stay int8 in LDS (half the DMA and LDS bytes) and become
//    bf16 in registers (exact: |q| <= 128 fits bf16's significand); the
//    per-channel scale is applied to the fp32 accumulator.
//
// LDS rows are dense with XOR-swizzled 16-byte chunks so that every
// fragment read (16 consecutive rows per quarter-wave) is bank-conflict
// free.  The k order inside a 32-wide k-tile is permuted identically for
// both operands (k-step st, lane half g reads k = 16 g + 8 st .. + 7), which
// lets one 16-byte read of an int8 row serve both k-steps.
#pragma once

#include "gemm_core.hpp"

namespace teeny {

// 16 zero bytes in device memory: the DMA source for rows past M / N and k
// past K, so that every k-tile issues the same number of DMA instructions.
__device__ __attribute__((aligned(16))) const uint32_t kGemmZero16[4] = {0u, 0u, 0u, 0u};

__device__ __forceinline__ uint32_t lds_address(const void *p) {
  typedef __attribute__((address_space(3))) const char lds_char;
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_char *)(p)));
}

// One 16-byte LDS-DMA per lane: lane j writes wave_lds + 16 j.  M0 carries
// the wave's LDS base and is restored afterwards.
__device__ __forceinline__ void lds_dma16(const void *src, uint32_t wave_lds) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(src), "s"(wave_lds)
      : "memory");
}

constexpr int kBigBM = 256, kBigBN = 256, kBigBK = 32, kBigStages = 4;

template <bool INT8B>
constexpr int big_stage_bytes() {
  return kBigBM * kBigBK * 2 + kBigBN * kBigBK * (INT8B ? 1 : 2);
}
template <bool INT8B>
constexpr int big_lds_bytes() {
  // pipeline stages, or the bf16 C tile of the epilogue, whichever is larger
  return kBigStages * big_stage_bytes<INT8B>() > kBigBM * (kBigBN + 8) * 2
             ? kBigStages * big_stage_bytes<INT8B>()
             : kBigBM * (kBigBN + 8) * 2;
}

template <bool INT8B, int AMODE>
__global__ __launch_bounds__(256, 1) void gemm_big_kernel(GemmParams p) {
  constexpr int BM = kBigBM, BN = kBigBN, BK = kBigBK, NST = kBigStages;
  constexpr int LA = 2;                                // DMA lookahead (k-tiles)
  constexpr int A_BYTES = BM * BK * 2;                 // 16 KiB
  constexpr int B_BYTES = BN * BK * (INT8B ? 1 : 2);   // 8 or 16 KiB
  constexpr int STAGE = A_BYTES + B_BYTES;
  constexpr int A_LD = A_BYTES / 16 / 256;             // DMA rounds per k-tile (A)
  constexpr int B_LD = B_BYTES / 16 / 256;             // DMA rounds per k-tile (B)
  constexpr int DMA_PER_KT = A_LD + B_LD;
  constexpr int MB = 4, NB = 4;                        // 32 x 32 blocks per wave
  static_assert(AMODE == kAPlain || AMODE == kAConvVec, "16-byte gather only");
  extern __shared__ __attribute__((aligned(16))) char smem[];

  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6, g = lane >> 5, c = lane & 31;
  const int wm = w >> 1, wn = w & 1;  // wave block: rows wm*128.. of m, wn*128.. of n

  const int tiles_m = (p.M + BM - 1) / BM;
  const int tile = xcd_remap(blockIdx.x, gridDim.x);
  const int m0 = (tile % tiles_m) * BM, n0 = (tile / tiles_m) * BN;
  const int n_k = (p.K + BK - 1) / BK;

  // ── DMA mapping.  A / bf16 B stage: 1024 slots of 16 B; slot t + 256 i is
  // row t / 4 + 64 i at chunk position t % 4 and holds data chunk
  // (t % 4) ^ ((t >> 4) & 3) (the row's swizzle, independent of i).
  // int8 B stage: 512 slots; slot t + 256 i is row t / 2 + 128 i at position
  // t % 2, data chunk (t % 2) ^ ((t >> 4) & 1).
  const int a_row0 = tid >> 2;
  const int a_col = ((tid & 3) ^ ((tid >> 4) & 3)) * 8;           // k offset (elements)
  const int b_row0 = INT8B ? (tid >> 1) : (tid >> 2);
  const int b_col = INT8B ? ((tid & 1) ^ ((tid >> 4) & 1)) * 16   // k offset (int8 elements)
                          : a_col;
  constexpr int B_RSTEP = INT8B ? 128 : 64;

  const bf16 *a_base[A_LD];
  bool a_ok[A_LD];
  int a_ih0[A_LD], a_iw0[A_LD];
#pragma unroll
  for (int i = 0; i < A_LD; ++i) {
    const int m = m0 + a_row0 + 64 * i;
    a_ok[i] = m < p.M;
    const int mm = a_ok[i] ? m : 0;
    if constexpr (AMODE == kAPlain) {
      a_base[i] = p.A + static_cast<int64_t>(mm) * p.lda;
      a_ih0[i] = a_iw0[i] = 0;
    } else {
      const int ow = mm % p.OW;
      const int t = mm / p.OW;
      const int oh = t % p.OH;
      const int b = t / p.OH;
      a_ih0[i] = oh * p.SH - p.PH;
      a_iw0[i] = ow * p.SW - p.PW;
      a_base[i] = p.A + static_cast<int64_t>(b) * p.H * p.W * p.Cin;
    }
  }
  // implicit-GEMM (kh, kw, ci) of this thread's chunk column, stepped by BK
  int k_ci = 0, k_kw = 0, k_kh = 0;
  if constexpr (AMODE == kAConvVec) {
    k_ci = a_col % p.Cin;
    const int r = a_col / p.Cin;
    k_kw = r % p.KW;
    k_kh = r / p.KW;
  }
  const uint32_t lds0 = lds_address(smem);
  // DMA instruction d (0 .. DMA_PER_KT-1) of k-tile kt into stage kt % NST
  // (zeros past n_k): d < A_LD are activation rounds, the rest weight rounds.
  // The activation gather of a conv needs this thread's (kh, kw, ci) for
  // k-tile kt: advance_k() steps it once the k-tile's A rounds are out.
  auto dma_one = [&](int kt, int d) __attribute__((always_inline)) {
    const uint32_t st_base = lds0 + (kt % NST) * STAGE;
    const int k0 = kt * BK;
    const bool live = kt < n_k;
    const void *src = kGemmZero16;
    uint32_t dst;
    if (d < A_LD) {
      const int i = d;
      const int k = k0 + a_col;
      if constexpr (AMODE == kAPlain) {
        if (live && a_ok[i] && k < p.K) src = a_base[i] + k;
      } else {
        const int ih = a_ih0[i] + k_kh, iw = a_iw0[i] + k_kw;
        if (live && a_ok[i] && k < p.K && ih >= 0 && ih < p.H && iw >= 0 && iw < p.W)
          src = a_base[i] + (static_cast<int64_t>(ih) * p.W + iw) * p.Cin + k_ci;
      }
      dst = st_base + i * 4096 + w * 1024;
    } else {
      const int i = d - A_LD;
      const int n = n0 + b_row0 + B_RSTEP * i;
      const int k = k0 + b_col;
      if (live && n < p.N && k < p.K) {
        if constexpr (INT8B)
          src = static_cast<const int8_t *>(p.B) + static_cast<int64_t>(n) * p.ldb + k;
        else
          src = static_cast<const bf16 *>(p.B) + static_cast<int64_t>(n) * p.ldb + k;
      }
      dst = st_base + A_BYTES + i * 4096 + w * 1024;
    }
    lds_dma16(src, __builtin_amdgcn_readfirstlane(dst));
  };
  auto advance_k = [&]() __attribute__((always_inline)) {
    if constexpr (AMODE == kAConvVec) {
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
  auto dma_tile = [&](int kt) __attribute__((always_inline)) {
#pragma unroll
    for (int d = 0; d < DMA_PER_KT; ++d) {
      dma_one(kt, d);
      if (d == A_LD - 1) advance_k();
    }
  };

  // ── fragment offsets (bytes within a stage).  Activations (B operand):
  // block j row wm*128 + 32 j + c, chunk 2 g + st at position
  // chunk ^ ((row >> 2) & 3) = chunk ^ ((c >> 2) & 3).  bf16 weights (A
  // operand) likewise with wn.  int8 weights: row wn*128 + 32 i + c, chunk g
  // at position g ^ ((c >> 3) & 1), 16 bytes = both k-steps.
  const int sw_a = (c >> 2) & 3;
  const int x_off = (wm * 128 + c) * 64;
  const int w_off = INT8B ? A_BYTES + (wn * 128 + c) * 32 + ((g ^ ((c >> 3) & 1)) << 4)
                          : A_BYTES + (wn * 128 + c) * 64;

  f32x16 acc[NB][MB];
#pragma unroll
  for (int i = 0; i < NB; ++i)
#pragma unroll
    for (int j = 0; j < MB; ++j) acc[i][j] = zero16();

  // A fragment set holds one k-tile: x[st][j] activations, w[st][i] bf16
  // weights (for int8, the converted weights).
  typedef bf16x8 frag_t;
  struct FragSet {
    frag_t x[2][MB];
    frag_t w[2][NB];
  };
  auto read_x = [&](const char *st_ptr, int st, int j, FragSet &f) __attribute__((always_inline)) {
    f.x[st][j] = *reinterpret_cast<const frag_t *>(st_ptr + x_off + j * 32 * 64 + (((2 * g + st) ^ sw_a) << 4));
  };
  auto read_w = [&](const char *st_ptr, int st, int i, FragSet &f) __attribute__((always_inline)) {
    f.w[st][i] = *reinterpret_cast<const frag_t *>(st_ptr + w_off + i * 32 * 64 + (((2 * g + st) ^ sw_a) << 4));
  };
  // int8: one 16-byte read per n-block covers both k-steps ...
  auto read_q = [&](const char *st_ptr, int i) __attribute__((always_inline)) {
    return *reinterpret_cast<const u32x4 *>(st_ptr + w_off + i * 32 * 32);
  };
  // ... and half of it (8 weights, one k-step) becomes one bf16 fragment
  auto convert_q = [&](const u32x4 &q, int st, int i, FragSet &f) __attribute__((always_inline)) {
    bf16 e[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int byte = 8 * st + t;
      const int8_t b = static_cast<int8_t>((q[byte >> 2] >> (8 * (byte & 3))) & 0xffu);
      e[t] = static_cast<bf16>(static_cast<float>(b));
    }
    __builtin_memcpy(&f.w[st][i], e, 16);
  };
  // One k-tile as 32 fenced bundles.  Bundle b issues MFMA (st, i, j) =
  // (b / 16, (b / 4) % 4, b % 4) plus a share of the other work: the DMA of
  // k-tile kt+3 (first bundles) and LDS reads that refill the single
  // fragment set in place: during the k-step-0 MFMAs the k-step-1 slots
  // (free since the previous k-tile) receive this k-tile's k-step-1
  // fragments; during the k-step-1 MFMAs the k-step-0 slots (just freed)
  // receive k-tile kt+1's (complete and published once tile kt starts).
  // int8 weights: one 16-byte read per n-block (q) serves both k-steps; its
  // k-step-0 half is converted for tile kt+1 during the second half and its
  // k-step-1 half during the first half of tile kt+1.
  FragSet f;
  u32x4 q[NB];
  auto ktile = [&](int kt) __attribute__((always_inline)) {
    const char *cu = smem + (kt % NST) * STAGE;
    const char *nx = smem + ((kt + 1) % NST) * STAGE;
    const bool more = kt + 1 < n_k;
#pragma unroll
    for (int b = 0; b < 32; ++b) {
      const int st = b >> 4, i = (b >> 2) & 3, j = b & 3;
      if (b < DMA_PER_KT) {
        dma_one(kt + 3, b);
        if (b == A_LD - 1) advance_k();
      }
      if (b < 16) {
        // this k-tile's k-step 1: MB activation reads (+ NB weight reads for bf16)
        if (b < MB) read_x(cu, 1, b, f);
        else if (!INT8B && b < MB + NB) read_w(cu, 1, b - MB, f);
      } else if (more) {
        // next k-tile's k-step 0 (int8: the weight chunks first)
        const int r = b - 16;
        if constexpr (INT8B) {
          if (r < NB) q[r] = read_q(nx, r);
          else if (r < NB + MB) read_x(nx, 0, r - NB, f);
        } else {
          if (r < MB) read_x(nx, 0, r, f);
          else if (r < MB + NB) read_w(nx, 0, r - MB, f);
        }
      }
      acc[i][j] = mfma32x32x16(f.w[st][i], f.x[st][j], acc[i][j]);
      if constexpr (INT8B) {
        // k-step-1 halves of this k-tile's chunks in bundles 4, 6, 8, 10;
        // k-step-0 halves of the next k-tile's in bundles 24, 26, 28, 30
        if (b >= 4 && b < 12 && (b & 1) == 0) convert_q(q[(b - 4) >> 1], 1, (b - 4) >> 1, f);
        if (more && b >= 24 && (b & 1) == 0) convert_q(q[(b - 24) >> 1], 0, (b - 24) >> 1, f);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // own DMA of earlier k-tiles complete (this k-tile's may still fly),
    // then the barrier that publishes them
    __builtin_amdgcn_s_waitcnt(0xF70 | DMA_PER_KT);
    __syncthreads();
  };

  // prologue: k-tiles 0..LA in flight, then all complete and published;
  // k-step 0 of k-tile 0 into the fragment set (int8: with its chunks in q)
#pragma unroll
  for (int t = 0; t <= LA; ++t) dma_tile(t);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
#pragma unroll
  for (int j = 0; j < MB; ++j) read_x(smem, 0, j, f);
  if constexpr (INT8B) {
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      q[i] = read_q(smem, i);
      convert_q(q[i], 0, i, f);
    }
  } else {
#pragma unroll
    for (int i = 0; i < NB; ++i) read_w(smem, 0, i, f);
  }
  for (int kt = 0; kt < n_k; ++kt) ktile(kt);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // trailing zero-source DMA
  __syncthreads();

  // ── epilogue: scale / bias / activation, bf16 C tile through LDS, 16-byte
  // row chunks out (coalesced).
  constexpr int CP = BN + 8;
  bf16 *cs = reinterpret_cast<bf16 *>(smem);
  // scale / bias per group of four columns (shared by the MB row blocks)
#pragma clang loop unroll(full)
  for (int i = 0; i < NB; ++i)
#pragma clang loop unroll(full)
    for (int v4 = 0; v4 < 4; ++v4) {
      float mul[4], add[4];
      epi_coeffs(p, n0 + wn * 128 + i * 32 + 8 * v4 + 4 * g, mul, add);
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
    const int ml = wm * 128 + j * 32 + c;
#pragma clang loop unroll(full)
    for (int i = 0; i < NB; ++i) {
#pragma clang loop unroll(full)
      for (int v4 = 0; v4 < 4; ++v4) {
        const int nl = wn * 128 + i * 32 + 8 * v4 + 4 * g;
        bf16x4 o4;
#pragma clang loop unroll(full)
        for (int e = 0; e < 4; ++e) {
          const float r = acc[i][j][4 * v4 + e];
          o4[e] = static_cast<bf16>(r < lo ? lo : r);
        }
        *reinterpret_cast<bf16x4 *>(cs + ml * CP + nl) = o4;
      }
    }
  }
  __syncthreads();
  constexpr int CPR_C = BN / 8;       // 16-byte chunks per C row
  constexpr int RPP_C = 256 / CPR_C;  // rows per pass
  const bool vec16 = (p.ldc % 8 == 0) && ((reinterpret_cast<uintptr_t>(p.C) & 15) == 0);
#pragma clang loop unroll(full)
  for (int r0 = 0; r0 < BM; r0 += RPP_C) {
    const int ml = r0 + tid / CPR_C, nl = (tid % CPR_C) * 8;
    const int m = m0 + ml, n = n0 + nl;
    if (m < p.M && n < p.N) {
      const u32x4 v = *reinterpret_cast<const u32x4 *>(cs + ml * CP + nl);
      bf16 *dst = p.C + static_cast<int64_t>(m) * p.ldc + n;
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

// Whether the large-tile kernel takes this problem: 16-byte chunks must
// never straddle a row or K (bf16: K % 8, int8: K % 16, 16-byte aligned
// operands and leading dimensions), the gather must be the vector one, N
// must fill a 256-wide tile, the k-loop must be long enough (K >= 512) for
// the pipeline to outweigh the 256 x 256 epilogue, and 256 x 256 tiles must
// still give every CU a workgroup.
template <bool INT8B, int AMODE>
inline bool big_gemm_fits(const GemmParams &p) {
  if (AMODE != kAPlain && AMODE != kAConvVec) return false;
  if (p.K % (INT8B ? 16 : 8) != 0 || p.K < 16 * kBigBK) return false;
  if (!aligned(p.A, 16) || !aligned(p.B, 16)) return false;
  if (AMODE == kAPlain && p.lda % 8 != 0) return false;
  if (p.ldb % (INT8B ? 16 : 8) != 0) return false;
  if (p.N < kBigBN) return false;  // narrower outputs would leave most of each tile idle
  return tiles_of(p, kBigBM, kBigBN) >= device_cu_count();
}

template <bool INT8B, int AMODE>
inline void launch_big_gemm(const GemmParams &p, hipStream_t s) {
  constexpr int bytes = big_lds_bytes<INT8B>();
  static const bool attr_set = [] {
    return hipFuncSetAttribute(reinterpret_cast<const void *>(&gemm_big_kernel<INT8B, AMODE>),
                               hipFuncAttributeMaxDynamicSharedMemorySize, bytes) == hipSuccess;
  }();
  (void)attr_set;
  const int grid = static_cast<int>(tiles_of(p, kBigBM, kBigBN));
  hipLaunchKernelGGL((gemm_big_kernel<INT8B, AMODE>), dim3(grid), dim3(256), bytes, s, p);
}

}  // namespace teeny
