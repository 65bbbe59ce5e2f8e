// Streaming GEMM for short K and narrow N with bf16 weights:
//
//   C[m, n] = act( scale[n] * sum_k A[m, k] * B[n, k] + bias[n] ),  K, N <= 256
//
// These are the 1x1 convolutions of a ResNet stage at full resolution
// (M = batch * H * W, e.g. 200,704 rows of 64 or 256 channels).  Their MFMA
// work is a few microseconds; A and C are 25-100 MB each, so the layer is
// bound by HBM traffic, and a tiled GEMM's per-tile prologue (first loads)
// and epilogue stretch it to about twice the copy time.  Here each
// workgroup stages all of B (N x K bf16, at most 64 KiB) and the per-column
// scale / bias in LDS once; then each of its waves walks its own
// sequence of 32-row blocks of A without further barriers:
//   * a block's rows arrive by LDS DMA, 1 KiB of consecutive bytes per
//     instruction (16-byte chunk k of row r lands at position k ^ (r % 8),
//     so the fragment reads below are free of bank conflicts), and the next
//     block's DMA is issued as soon as the current block's fragments are in
//     registers, so it overlaps the MFMAs and the epilogue;
//   * v_mfma_f32_32x32x16_bf16 computes C^T (B fragments from LDS as the A
//     operand, A rows as the B operand): a lane's accumulator column is one
//     output row m and four consecutive registers are four consecutive n;
//     a lane swap across the wave halves (v_permlane32_swap) makes eight
//     consecutive n per lane;
//   * the outputs pass through a 4 KiB per-wave LDS slice, 64 columns at a
//     time, and leave as stores of 1 KiB runs of whole rows (16-byte stores
//     of 32 different rows reach about 60 % of the write bandwidth).
// Rows past M load and store through buffer resources at an offset past
// their extent (zeros, no memory traffic; stores dropped).
#pragma once

#include <atomic>
#include <type_traits>

namespace teeny {

// Waves per workgroup.  A wave keeps one 32-row block of A in flight while
// it computes the previous one, and at these sizes the layer is bound by the
// bytes in flight per CU (about 16 KiB per wave against HBM latency), so a
// workgroup takes as many waves as its LDS holds beside B (one 32 x K A
// slice and one 4 KiB output slice per wave) and as the registers allow (an
// estimate of N/2 accumulator, K/4 fragment and 32 other registers per lane,
// against 512 per SIMD lane).  Measured on MI355X against four-wave
// workgroups, the stage-1 1x1 convs of ResNet-50 at batch 64: 64 -> 64
// 11.4 -> 10.3 us, 256 -> 64 25.8 -> 25.3 us, 64 -> 256 26-28 -> 25-29 us
// (eight waves either way; the 53-conv step 1.501 -> 1.485 ms).  The
// gain is small: bytes in flight are not the main limit of these layers.
constexpr int stream_waves(int K, int N) {
  const int by_lds = (160 * 1024 - N * (K + 8) * 2 - 2 * N * 4) / (32 * K * 2 + 32 * 64 * 2);
  const int by_regs = 4 * (512 / (N / 2 + K / 4 + 32));
  const int w = by_lds < by_regs ? by_lds : by_regs;
  return w < 16 ? w : 16;
}

template <int K, int N>
__global__ __launch_bounds__(64 * stream_waves(K, N), 1) void gemm_stream_kernel(GemmParams p) {
  constexpr int WV = stream_waves(K, N);
  constexpr int KS = K / 16;         // MFMA k-steps
  constexpr int NB = N / 32;         // 32-column output blocks
  constexpr int KP = K + 8;          // LDS pitch of a B row (elements): 16-byte reads of 8 rows hit disjoint banks
  constexpr int ACH = K / 8;         // 16-byte chunks per A row
  constexpr int NI = 32 * ACH / 64;  // DMA instructions per block (64 chunks each)
  constexpr int A_STG = 32 * K * 2;  // bytes of one wave's A block
  constexpr int C_STG = 32 * 64 * 2; // bytes of one wave's output slice (64 columns)
  static_assert(K % 64 == 0 && N % 64 == 0 && K <= 256 && N <= 256, "stream GEMM shape");
  __shared__ __attribute__((aligned(16))) bf16 bs[N * KP];
  __shared__ __attribute__((aligned(16))) float cmul[N];
  __shared__ __attribute__((aligned(16))) float cadd[N];
  __shared__ __attribute__((aligned(16))) char stg[WV * (A_STG + C_STG)];

  const int tid = threadIdx.x;
  const int lane = tid & 63, g = lane >> 5, c = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar block loop
  char *const a_stg = stg + w * (A_STG + C_STG);
  char *const c_stg = a_stg + A_STG;
  const uint32_t a_lds = __builtin_amdgcn_readfirstlane(lds_address(a_stg));

  const int nblk = (p.M + 31) / 32;
  const int stride = static_cast<int>(gridDim.x) * WV;
  int blk = static_cast<int>(blockIdx.x) * WV + w;
  const __amdgpu_buffer_rsrc_t a_rsrc = buffer_rsrc(p.A, p.a_bytes);
  const __amdgpu_buffer_rsrc_t c_rsrc = buffer_rsrc(p.C, static_cast<int>((static_cast<int64_t>(p.M - 1) * p.ldc + N) * 2));
  // DMA of block b: instruction i, lane j fills LDS chunk 64 i + j = row r,
  // position r * ACH + q with global chunk q ^ (r % 8)
  auto dma = [&](int b) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int slot = 64 * i + lane;
      const int r = slot / ACH, q = slot % ACH;
      const int m = b * 32 + r;
      const int off = m < p.M ? static_cast<int>(static_cast<int64_t>(m) * p.lda * 2) + 16 * (q ^ (r & 7)) : kOffNone;
      buffer_lds_dma16(a_rsrc, off, a_lds + 1024 * i);
    }
  };
  // the first block's DMA goes out before the prologue; a wave without
  // blocks issues none (it must not leave DMA writes pending when it ends)
  if (blk < nblk) dma(blk);

  // ── prologue: B and the epilogue coefficients into LDS ──────────────
  constexpr int CPR = K / 8;  // 16-byte chunks per B row
  const bf16 *B = static_cast<const bf16 *>(p.B);
  for (int i = tid; i < N * CPR; i += 64 * WV) {
    const int n = i / CPR, j = i % CPR;
    *reinterpret_cast<u32x4 *>(bs + n * KP + 8 * j) =
        *reinterpret_cast<const u32x4 *>(B + static_cast<int64_t>(n) * p.ldb + 8 * j);
  }
  for (int n = tid; n < N; n += 64 * WV) {
    float m = 1.0f, a = 0.0f;
    if (p.scale != nullptr) m = p.scale[n];
    if (p.bias != nullptr) a = p.bias[n];
    if (p.bias_bf16 != nullptr) a += static_cast<float>(p.bias_bf16[n]);
    cmul[n] = m;
    cadd[n] = a;
  }
  __syncthreads();
  if (blk >= nblk) return;  // no barrier follows; this wave issued no DMA

  const EpiAct ea = epi_act(p.act);
  const float lo = ea.relu ? 0.0f : -INFINITY;
  auto bfrag = [&](int s, int j) __attribute__((always_inline)) {
    return *reinterpret_cast<const bf16x8 *>(bs + (32 * j + c) * KP + 16 * s + 8 * g);
  };
  for (;;) {
    // block blk's DMA (and the previous block's stores) complete
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    // A fragments: lane (c, g), step s: row c, chunk 2 s + g
    bf16x8 af[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s)
      af[s] = *reinterpret_cast<const bf16x8 *>(a_stg + c * (K * 2) + 16 * ((2 * s + g) ^ (c & 7)));
    // the reads are done before the next DMA overwrites the slice
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    const int nb = blk + stride;
    if (nb < nblk) dma(nb);

    f32x16 acc[NB];
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[j] = zero16();
    // B fragments are read one step ahead of their MFMA.  The empty asm
    // with a memory clobber after each MFMA keeps every read inside its
    // block: the fragments are loop-invariant, and hoisting all of them out
    // of the block loop (or ahead of the MFMAs) would hold N * K / 32
    // registers instead of two fragments.
    bf16x8 bn = bfrag(0, 0);
#pragma unroll
    for (int s = 0; s < KS; ++s) {
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        const bf16x8 b = bn;
        if (j + 1 < NB) bn = bfrag(s, j + 1);
        else if (s + 1 < KS) bn = bfrag(s + 1, 0);
        acc[j] = mfma32x32x16(b, af[s], acc[j]);
        asm volatile("" ::: "memory");
      }
    }

    // Epilogue, 64 columns (j = 2 h, 2 h + 1) at a time.  Register group q
    // of lane half g holds columns 32 j + 8 q + 4 g + (0..3); one
    // v_permlane32_swap per dword trades the odd group of the lower half for
    // the even group of the upper half, so lane (c, g) holds the 16-byte
    // chunk 4 (j % 2) + 2 pr + g of the slice, row c.
    const int m0 = blk * 32;
    auto epilogue = [&](auto sig) __attribute__((always_inline)) {
#pragma unroll
      for (int h = 0; h < NB / 2; ++h) {
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
          const int j = 2 * h + jj;
#pragma unroll
          for (int pr = 0; pr < 2; ++pr) {
            u32x2 hv[2];
#pragma unroll
            for (int t = 0; t < 2; ++t) {
              const int q = 2 * pr + t;
              const int n = 32 * j + 8 * q + 4 * g;
              const f32x4 mul = *reinterpret_cast<const f32x4 *>(cmul + n);
              const f32x4 add = *reinterpret_cast<const f32x4 *>(cadd + n);
              bf16x4 o;
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                float r = __builtin_fmaf(acc[j][4 * q + e], mul[e], add[e]);
                if constexpr (decltype(sig)::value) r = epi_sig(r, ea);
                o[e] = static_cast<bf16>(r < lo ? lo : r);
              }
              hv[t] = __builtin_bit_cast(u32x2, o);
            }
            u32x4 v;
#pragma unroll
            for (int d = 0; d < 2; ++d) {
              const auto sw = __builtin_amdgcn_permlane32_swap(hv[0][d], hv[1][d], false, false);
              v[d] = sw[0];
              v[2 + d] = sw[1];
            }
            const int k = 4 * jj + 2 * pr + g;
            *reinterpret_cast<u32x4 *>(c_stg + c * 128 + 16 * (k ^ (c & 7))) = v;
          }
        }
        // the slice back as whole 128-byte row segments: instruction i, lane
        // L holds row 8 i + L / 8, position L % 8 = column chunk (L % 8) ^ (row % 8),
        // by non-temporal stores (cache policy nt): on the 56x56 ResNet 1x1
        // convs 64 -> 256 26.8 -> 24.3 us, 256 -> 64 25.3 -> 24.7 us, the
        // step 1.278 -> 1.274 ms; non-temporal A loads as well cost the
        // layers alone ~10 %
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = 8 * i + (lane >> 3), pos = lane & 7;
          const u32x4 v = *reinterpret_cast<const u32x4 *>(c_stg + r * 128 + 16 * pos);
          const int m = m0 + r;
          const int off = m < p.M ? static_cast<int>(static_cast<uint32_t>(m) * static_cast<uint32_t>(p.ldc) * 2u) +
                                        2 * 64 * h + 16 * (pos ^ (r & 7))
                                  : kOffNone;
          __builtin_amdgcn_raw_buffer_store_b128(v, c_rsrc, off, 0, 2);
        }
      }
    };
    if (ea.sig) epilogue(std::true_type{});
    else epilogue(std::false_type{});
    blk = nb;
    if (blk >= nblk) break;
  }
}

// Shapes the streaming kernel is instantiated for, and its preconditions:
// plain bf16 A with 16-byte aligned rows, bf16 B with 16-byte aligned rows,
// C rows 16-byte aligned (the epilogue writes 16-byte chunks at row offsets
// m * ldc * 2 + 16 j, so both C and ldc * 2 must be multiples of 16), and
// enough rows that the problem is bound by HBM traffic (below that the tiled
// kernels are as fast).
constexpr int kStreamMinM = 16384;
inline bool stream_shape(int K, int N) {
  return (K == 64 || K == 128 || K == 256) && (N == 64 || N == 128 || N == 256) && N * K <= 32768;
}
template <bool INT8B, int AMODE>
inline bool stream_gemm_fits(const GemmParams &p) {
  if constexpr (INT8B || AMODE != kAPlain) {
    return false;
  } else {
    return stream_shape(p.K, p.N) && p.M >= kStreamMinM && static_cast<int64_t>(p.M) * p.ldc * 2 < 0x7fffffff &&
           p.lda % 8 == 0 && p.ldb % 8 == 0 &&
           p.ldc % 8 == 0 && (reinterpret_cast<uintptr_t>(p.A) & 15) == 0 &&
           (reinterpret_cast<uintptr_t>(p.B) & 15) == 0 && (reinterpret_cast<uintptr_t>(p.C) & 15) == 0;
  }
}

template <int K, int N>
inline void launch_stream_kn(const GemmParams &p, hipStream_t s) {
  constexpr int WV = stream_waves(K, N);
  // resident workgroups per CU, cached per device ordinal (relaxed atomics:
  // racing threads compute and store the same value)
  static std::atomic<int> occupancy[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = -1;
  int per_cu = dev >= 0 ? occupancy[dev].load(std::memory_order_relaxed) : 0;
  if (per_cu <= 0) {
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, gemm_stream_kernel<K, N>, 64 * WV, 0) != hipSuccess ||
        per_cu < 1)
      per_cu = 1;
    if (dev >= 0) occupancy[dev].store(per_cu, std::memory_order_relaxed);
  }
  // Every wave walks the same number of blocks (the last round of a
  // ragged split would run a small fraction of the waves alone).
  const int64_t nblk = (p.M + 31) / 32;
  const int64_t slots = static_cast<int64_t>(per_cu) * device_cu_count() * WV;
  const int64_t per_wave = (nblk + slots - 1) / slots;
  const int64_t grid = ((nblk + per_wave - 1) / per_wave + WV - 1) / WV;
  hipLaunchKernelGGL((gemm_stream_kernel<K, N>), dim3(static_cast<unsigned>(grid)), dim3(64 * WV), 0, s, p);
}

inline void launch_stream_gemm(const GemmParams &p, hipStream_t s) {
  switch (p.K * 1000 + p.N) {
    case 64064: launch_stream_kn<64, 64>(p, s); break;
    case 64128: launch_stream_kn<64, 128>(p, s); break;
    case 64256: launch_stream_kn<64, 256>(p, s); break;
    case 128064: launch_stream_kn<128, 64>(p, s); break;
    case 128128: launch_stream_kn<128, 128>(p, s); break;
    case 128256: launch_stream_kn<128, 256>(p, s); break;
    case 256064: launch_stream_kn<256, 64>(p, s); break;
    default: launch_stream_kn<256, 128>(p, s); break;
  }
}

}  // namespace teeny
