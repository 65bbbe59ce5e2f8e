// Persistent LDS-DMA GEMM: one pipeline per workgroup across all its tiles.
//
//   C[m, n] = act( scale[n] * sum_k A[m, k] * B[n, k] + bias[n] )
//
// Same contract, operand staging and k-tile schedule as gemm_dma_kernel
// (bf16 operands, A plain or the NHWC implicit-GEMM gather).  The
// difference is the tile loop: the grid is the number of workgroups the
// chip holds at once, and each workgroup multiplies tiles wg, wg + G,
// wg + 2G, ... with ONE LDS-DMA ring that runs NST-1 k-tiles ahead of the
// MFMAs regardless of tile boundaries.  While a tile's last k-tiles are
// multiplied, the DMA already fetches the next tile's first ones, and the
// epilogue (scale, bias, activation, bf16 rows written back through the LDS
// stage the tile's last k-tile just freed) runs while those land.  For the mid-sized convolutions of a
// ResNet (K of 128 .. 1152, a few tiles per CU) a tile otherwise pays its
// first loads' full memory latency and its epilogue with the k-loop stalled.
//
// The DMA cursor (tile position, k-tile) advances one k-tile per k-tile of
// MFMA work; when it reaches the next tile it recomputes its row offsets
// (the conv gather decodes (b, oh, ow) per row) and restarts the tap walk.
// Past the workgroup's last tile it issues zero-source DMAs, so every
// k-tile issues the same DMA count and the explicit vmcnt waits stay exact.
// The epilogue's stores are compiler-visible buffer stores; the kernel's own
// waits count them in issue order with the DMAs (the first k-tile after an
// epilogue allows for them).  Each store instruction writes eight
// whole 128-byte row segments: stores of 8 bytes per lane straight from the
// accumulators (32 rows x 16 bytes per instruction) wrote at ~1.4 TB/s and
// took more time than the whole k-loop on the 1x1 convs.
#pragma once

#include <atomic>
#include <type_traits>

namespace teeny {

// Widest N the kernel takes: the epilogue coefficients of every column sit
// in LDS (2 x 8 KiB).
constexpr int kPersistMaxN = 2048;

template <int BM, int BN, int NST, int MINW, int AMODE>
__global__ __launch_bounds__(256, MINW) void gemm_persist_kernel(GemmParams p) {
  constexpr int BK = kDmaBK;
  constexpr int WM = BM / 2, WN = BN / 2;  // wave block (2 x 2 waves)
  constexpr int MB = WM / 32, NB = WN / 32;
  constexpr int H = MB * NB;
  constexpr int A_BYTES = BM * BK * 2;
  constexpr int B_BYTES = BN * BK * 2;
  constexpr int STAGE = A_BYTES + B_BYTES;
  constexpr int A_LD = A_BYTES / 16 / 256;
  constexpr int B_LD = B_BYTES / 16 / 256;
  constexpr int DMA_PER_KT = A_LD + B_LD;
  constexpr int INFLIGHT = DMA_PER_KT * (NST - 3);
  static_assert(AMODE == kAPlain || AMODE == kAConvVec, "16-byte gather only");
  static_assert(A_BYTES % 4096 == 0 && B_BYTES % 4096 == 0, "whole DMA rounds per k-tile");
  static_assert(MB >= 2 && NB >= 2 && MB + NB <= H && DMA_PER_KT <= 2 * H, "bundle schedule");
  static_assert(NST >= 4 && INFLIGHT < 16, "stages / vmcnt field");
  static_assert(NB == 2 && STAGE >= 4 * 4096, "epilogue: 64-column wave blocks, a 4 KiB slice per wave");
  extern __shared__ __attribute__((aligned(16))) char smem[];

  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6, g = lane >> 5, c = lane & 31;
  const int wm = w >> 1, wn = w & 1;

  const int tiles_m = (p.M + BM - 1) / BM;
  const int tiles_n = (p.N + BN - 1) / BN;
  const int n_tiles = tiles_m * tiles_n;
  const int G = static_cast<int>(gridDim.x);
  const int wg = xcd_remap(blockIdx.x, G);
  const int my_tiles = wg < n_tiles ? (n_tiles - 1 - wg) / G + 1 : 0;
  const int n_k = (p.K + BK - 1) / BK;
  const bool n_fast = p.n_fast != 0;
  auto tile_origin = [&](int pos, int &m0, int &n0) __attribute__((always_inline)) {
    const int t = wg + pos * G;
    const int tm = n_fast ? t / tiles_n : t % tiles_m;
    const int tn = n_fast ? t % tiles_n : t / tiles_m;
    m0 = tm * BM;
    n0 = tn * BN;
  };

  // ── DMA side (see gemm_dma_kernel for the slot mapping) ───────────────
  const int a_row0 = tid >> 2;
  const int a_col = ((tid & 3) ^ ((tid >> 4) & 3)) * 8;
  const int b_row0 = tid >> 2;
  const int b_col = a_col;
  const __amdgpu_buffer_rsrc_t a_rsrc = buffer_rsrc(p.A, p.a_bytes);
  const __amdgpu_buffer_rsrc_t b_rsrc = buffer_rsrc(p.B, p.b_bytes);
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
    t.off = 2 * ((t.kh * p.W + t.kw) * p.Cin + t.ci);
    return t;
  };
  auto tap_step = [&](TapState &t, bool once) __attribute__((always_inline)) {
    t.ci += BK;
    t.off += 2 * BK;
    while (t.ci >= p.Cin) {
      t.ci -= p.Cin;
      if (++t.kw == p.KW) {
        t.kw = 0;
        ++t.kh;
        t.off += 2 * (p.W - p.KW) * p.Cin;
      }
      if (once) break;
    }
  };
  // cursor: tile position d_pos of this workgroup, k-tile d_kt of it,
  // global k-tile count d_gk (selects the LDS stage)
  int d_pos = 0, d_kt = 0, d_gk = 0;
  int a_off[A_LD], a_ih0[A_LD], a_iw0[A_LD], b_off[B_LD];
  // tap walk: of the k-tile's first column when C_IN % BK == 0 (then a
  // k-tile never straddles a tap and the thread adds its column), else of
  // the thread's own column
  TapState tap{0, 0, 0, 0};
  const int tap_col_bytes = tap_uniform ? 2 * a_col : 0;
  auto dma_setup = [&]() __attribute__((always_inline)) {
    int m0 = 0, n0 = 0;
    if (d_pos < my_tiles) tile_origin(d_pos, m0, n0);
#pragma unroll
    for (int i = 0; i < A_LD; ++i) {
      const int m = min(m0 + a_row0 + 64 * i, p.M - 1);
      if constexpr (AMODE == kAPlain) {
        a_off[i] = static_cast<int>(static_cast<int64_t>(m) * p.lda * 2);
        a_ih0[i] = a_iw0[i] = 0;
      } else {
        const int ow = m % p.OW;
        const int t = m / p.OW;
        const int oh = t % p.OH;
        const int b = t / p.OH;
        a_ih0[i] = oh * p.SH - p.PH;
        a_iw0[i] = ow * p.SW - p.PW;
        a_off[i] = static_cast<int>(2 * (static_cast<int64_t>(b) * p.H * p.W * p.Cin +
                                         static_cast<int64_t>(a_ih0[i] * p.W + a_iw0[i]) * p.Cin));
      }
    }
#pragma unroll
    for (int i = 0; i < B_LD; ++i) {
      const int n = min(n0 + b_row0 + 64 * i, p.N - 1);
      b_off[i] = static_cast<int>(static_cast<int64_t>(n) * p.ldb * 2);
    }
    if constexpr (AMODE == kAConvVec) tap = tap_at(tap_uniform ? 0 : a_col);
  };
  const uint32_t lds0 = lds_address(smem);
  // DMA instruction d of the cursor's k-tile into stage d_gk % NST
  auto dma_one = [&](int d) __attribute__((always_inline)) {
    const uint32_t st_base = lds0 + (d_gk % NST) * STAGE;
    const int k0 = d_kt * BK;
    const bool live = d_pos < my_tiles;
    if (d < A_LD) {
      const int i = d;
      const int k = k0 + a_col;
      int off;
      if constexpr (AMODE == kAPlain) {
        off = (live & (k < p.K)) ? a_off[i] + 2 * k : kOffNone;
      } else {
        const int ih = a_ih0[i] + tap.kh, iw = a_iw0[i] + tap.kw;
        const bool ok = live & (k < p.K) & (static_cast<unsigned>(ih) < static_cast<unsigned>(p.H)) &
                        (static_cast<unsigned>(iw) < static_cast<unsigned>(p.W));
        off = ok ? a_off[i] + tap.off + tap_col_bytes : kOffNone;
      }
      buffer_lds_dma16(a_rsrc, off, __builtin_amdgcn_readfirstlane(st_base + i * 4096 + w * 1024));
    } else {
      const int i = d - A_LD;
      const int k = k0 + b_col;
      const int off = (live & (k < p.K)) ? b_off[i] + 2 * k : kOffNone;
      buffer_lds_dma16(b_rsrc, off, __builtin_amdgcn_readfirstlane(st_base + A_BYTES + i * 4096 + w * 1024));
    }
  };
  // after a k-tile's DMAs: the next k-tile of the tile, or the next tile
  auto dma_advance = [&]() __attribute__((always_inline)) {
    ++d_gk;
    if (++d_kt == n_k) {
      d_kt = 0;
      ++d_pos;
      dma_setup();
    } else if constexpr (AMODE == kAConvVec) {
      tap_step(tap, tap_uniform);
    }
  };

  // ── MFMA side ─────────────────────────────────────────────────────────
  const int sw_a = (c >> 2) & 3;
  const int x_off = (wm * WM + c) * 64;
  const int w_off = A_BYTES + (wn * WN + c) * 64;
  f32x16 acc[NB][MB];
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
  FragSet f;
  // k-tile gk (stage gk % NST): 2H fenced bundles, each one MFMA, the first
  // DMA_PER_KT of them also one DMA of the cursor's k-tile; the fragment
  // set is refilled in place (k-step 1 of this k-tile during the k-step-0
  // MFMAs, k-step 0 of k-tile gk+1 during the k-step-1 MFMAs)
  // Stores of one epilogue per wave (MB row blocks x 4 instructions).  The
  // first k-tile after an epilogue waits for the DMA issued before those
  // stores, so its count includes them (vector memory operations retire in
  // issue order): the stores stay in flight instead of being drained.
  constexpr int EPI_STORES = MB * 4;
  static_assert(INFLIGHT + EPI_STORES < 16, "vmcnt field");
  auto ktile = [&](int gk, bool after_epilogue) __attribute__((always_inline)) {
    const char *cu = smem + (gk % NST) * STAGE;
    const char *nx = smem + ((gk + 1) % NST) * STAGE;
#pragma unroll
    for (int b = 0; b < 2 * H; ++b) {
      const int st = b / H, i = (b % H) / MB, j = b % MB;
      if (b < DMA_PER_KT) dma_one(b);
      if (b < H) {
        if (b < MB) read_x(cu, 1, b, f);
        else if (b < MB + NB) read_w(cu, 1, b - MB, f);
      } else {
        const int r = b - H;
        if (r < MB) read_x(nx, 0, r, f);
        else if (r < MB + NB) read_w(nx, 0, r - MB, f);
      }
      acc[i][j] = mfma32x32x16(f.w[st][i], f.x[st][j], acc[i][j]);
      __builtin_amdgcn_sched_barrier(0);
    }
    dma_advance();
    if (after_epilogue) __builtin_amdgcn_s_waitcnt(0xF70 | (INFLIGHT + EPI_STORES));
    else __builtin_amdgcn_s_waitcnt(0xF70 | INFLIGHT);
    __syncthreads();
  };

  // Epilogue coefficients: mul = scale (or 1) and add = bias (fp32 and/or
  // bf16, or 0) for every column, staged in LDS once (filled after the
  // prologue's DMAs are issued, so both latencies overlap).  A global load
  // in the tile loop would make the compiler wait with vmcnt(0), which also
  // waits for every DMA in flight.
  float *const cmul = reinterpret_cast<float *>(smem + NST * STAGE);
  float *const cadd = cmul + kPersistMaxN;

  const EpiAct ea = epi_act(p.act);
  const float lo = ea.relu ? 0.0f : -INFINITY;
  const __amdgpu_buffer_rsrc_t c_rsrc =
      buffer_rsrc(p.C, static_cast<int>((static_cast<int64_t>(p.M - 1) * p.ldc + p.N) * 2));
  // Epilogue of the tile at (m0, n0), run right after its last k-tile,
  // whose LDS stage `slot` is free until the next k-tile's DMA: each wave
  // stages its 64 x 64 block there, 32 rows (one row block j) at a time, in
  // a 4 KiB slice of its own, and writes it back as whole 128-byte row
  // segments (one store instruction = 8 full rows of the block).  Register
  // group q of lane half g holds columns 32 i + 8 q + 4 g + (0..3); one
  // v_permlane32_swap per dword trades the odd group of the lower half for
  // the even group of the upper half, so lane (c, g) holds the 16-byte chunk
  // 4 i + 2 pr + g of row c.
  auto epilogue = [&](int m0, int n0, int slot, auto sig, auto scaled) __attribute__((always_inline)) {
    char *const c_stg = smem + slot * STAGE + w * 4096;
    const int nw = n0 + wn * WN;  // the wave's first column
    // the wave's 64 coefficients (x 2 with a scale), read as one batch
    // (read one by one next to their uses, each read was waited for on its
    // own)
    f32x4 mulv[NB][4], addv[NB][4];
#pragma clang loop unroll(full)
    for (int i = 0; i < NB; ++i)
#pragma clang loop unroll(full)
      for (int q = 0; q < 4; ++q) {
        const int nc = min(nw + 32 * i + 8 * q + 4 * g, kPersistMaxN - 4);
        if constexpr (decltype(scaled)::value) mulv[i][q] = *reinterpret_cast<const f32x4 *>(cmul + nc);
        else mulv[i][q] = f32x4{1.0f, 1.0f, 1.0f, 1.0f};
        addv[i][q] = *reinterpret_cast<const f32x4 *>(cadd + nc);
      }
    __builtin_amdgcn_sched_barrier(0);
#pragma clang loop unroll(full)
    for (int j = 0; j < MB; ++j) {
#pragma clang loop unroll(full)
      for (int i = 0; i < NB; ++i) {
#pragma clang loop unroll(full)
        for (int pr = 0; pr < 2; ++pr) {
          u32x2 hv[2];
#pragma clang loop unroll(full)
          for (int t = 0; t < 2; ++t) {
            const int q = 2 * pr + t;
            const f32x4 mul = mulv[i][q], add = addv[i][q];
            bf16x4 o;
#pragma clang loop unroll(full)
            for (int e = 0; e < 4; ++e) {
              float r = __builtin_fmaf(acc[i][j][4 * q + e], mul[e], add[e]);
              if constexpr (decltype(sig)::value) r = epi_sig(r, ea);
              o[e] = static_cast<bf16>(r < lo ? lo : r);
            }
            hv[t] = __builtin_bit_cast(u32x2, o);
          }
          u32x4 v;
#pragma clang loop unroll(full)
          for (int d = 0; d < 2; ++d) {
            const auto sw = __builtin_amdgcn_permlane32_swap(hv[0][d], hv[1][d], false, false);
            v[d] = sw[0];
            v[2 + d] = sw[1];
          }
          const int k = 4 * i + 2 * pr + g;
          *reinterpret_cast<u32x4 *>(c_stg + c * 128 + 16 * (k ^ (c & 7))) = v;
        }
      }
      // rows back as 128-byte segments: instruction r8, lane L holds row
      // 8 r8 + L / 8, position L % 8 = column chunk (L % 8) ^ (row % 8), by
      // non-temporal stores (cache policy nt), which leave the caches to the
      // DMA ring's operands: 200704 x 128 x 256 35.7 -> 28.0 us, the stage-3
      // 1x1 convs 17.9 -> 15.2 us, the ResNet step 1.278 -> 1.257 ms
#pragma clang loop unroll(full)
      for (int r8 = 0; r8 < 4; ++r8) {
        const int r = 8 * r8 + (lane >> 3), pos = lane & 7;
        const u32x4 v = *reinterpret_cast<const u32x4 *>(c_stg + r * 128 + 16 * pos);
        const int m = m0 + wm * WM + 32 * j + r;
        const int off = ((m < p.M) & (nw < p.N))
                            ? static_cast<int>((static_cast<uint32_t>(m) * static_cast<uint32_t>(p.ldc) +
                                                static_cast<uint32_t>(nw)) * 2u) + 16 * (pos ^ (r & 7))
                            : kOffNone;
        __builtin_amdgcn_raw_buffer_store_b128(v, c_rsrc, off, 0, 2);
      }
    }
  };

  // prologue: the first NST-1 k-tiles in flight, 0 and 1 complete
  dma_setup();
#pragma unroll
  for (int t = 0; t < NST - 1; ++t) {
#pragma unroll
    for (int d = 0; d < DMA_PER_KT; ++d) dma_one(d);
    dma_advance();
  }
  for (int n = tid; n < kPersistMaxN; n += 256) {
    float m = 1.0f, a = 0.0f;
    if (n < p.N) {
      if (p.scale != nullptr) m = p.scale[n];
      if (p.bias != nullptr) a = p.bias[n];
      if (p.bias_bf16 != nullptr) a += static_cast<float>(p.bias_bf16[n]);
    }
    cmul[n] = m;
    cadd[n] = a;
  }
  __builtin_amdgcn_s_waitcnt(0xF70 | INFLIGHT);
  __syncthreads();
#pragma unroll
  for (int j = 0; j < MB; ++j) read_x(smem, 0, j, f);
#pragma unroll
  for (int i = 0; i < NB; ++i) read_w(smem, 0, i, f);

  int gk = 0;
  for (int pos = 0; pos < my_tiles; ++pos) {
#pragma unroll
    for (int i = 0; i < NB; ++i)
#pragma unroll
      for (int j = 0; j < MB; ++j) acc[i][j] = zero16();
    for (int kt = 0; kt < n_k; ++kt) ktile(gk++, kt == 0 && pos > 0);
    int m0, n0;
    tile_origin(pos, m0, n0);
    const int slot = (gk - 1) % NST;  // the stage of the tile's last k-tile
    if (p.scale != nullptr) {
      if (ea.sig) epilogue(m0, n0, slot, std::true_type{}, std::true_type{});
      else epilogue(m0, n0, slot, std::false_type{}, std::true_type{});
    } else {
      if (ea.sig) epilogue(m0, n0, slot, std::true_type{}, std::false_type{});
      else epilogue(m0, n0, slot, std::false_type{}, std::false_type{});
    }
    // the slot's next DMA is issued by the next k-tile
    __syncthreads();
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // trailing zero-source DMA
}

template <int BM, int BN, int NST>
constexpr int persist_lds_bytes() {
  return NST * (BM + BN) * kDmaBK * 2 + 2 * kPersistMaxN * 4;
}

// Grid: the workgroups the chip holds at once (or fewer when there are
// fewer tiles).
template <int BM, int BN, int NST, int MINW, int AMODE>
inline void launch_persist_gemm(const GemmParams &p, hipStream_t s, int max_grid = 0) {
  constexpr int bytes = persist_lds_bytes<BM, BN, NST>();
  auto kern = &gemm_persist_kernel<BM, BN, NST, MINW, AMODE>;
  static const bool attr_set = [kern] {
    return hipFuncSetAttribute(reinterpret_cast<const void *>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                               bytes) == hipSuccess;
  }();
  (void)attr_set;
  static std::atomic<int> occupancy[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = -1;
  int per_cu = dev >= 0 ? occupancy[dev].load(std::memory_order_relaxed) : 0;
  if (per_cu <= 0) {
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, 256, bytes) != hipSuccess || per_cu < 1)
      per_cu = 1;
    if (dev >= 0) occupancy[dev].store(per_cu, std::memory_order_relaxed);
  }
  const int64_t tiles = tiles_of(p, BM, BN);
  int64_t grid = std::min<int64_t>(tiles, static_cast<int64_t>(per_cu) * device_cu_count());
  if (max_grid > 0) grid = std::min<int64_t>(grid, max_grid);
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(grid)), dim3(256), bytes, s, p);
}

// When the tile policy takes the persistent kernel: bf16 operands that the
// LDS DMA can read (dma_gemm_ok), N a multiple of the 128-column tile up to
// kPersistMaxN (narrower outputs waste tile columns: the 64-channel stem GEMM
// ran 74 -> 124 us), C rows 16-byte aligned with
// 32-bit byte offsets, and a problem of many tiles with a short k-loop:
// >= 1.5 tiles of 128 x 128 per CU and K of 128 .. 512 (.. 1024 for N <=
// 1024).  Measured on MI355X (batch-64 ResNet-50 convs): 200704 x 128 x 256
// 43.6 -> 37.4 us (against the streaming kernel), 50176 x 512 x 128 23.5 ->
// 20.5 us, 50176 x 512 x 256 (stride-2 1x1) 34.0 -> 30.6 us; with each conv
// reading the previous one's output, the stage-3 1x1 convs (784 tiles)
// 20.9 -> 18.6 us, 50176 x 256 x 512 29.3 -> 26.5 us, 12544 x 512 x 1024
// 24.6 -> 23.0 us (the ResNet step 1.332 -> 1.312 ms); 3136 x 2048 x 1024
// (strided 1x1) 25.7 -> 27.5 us and deep K (40 vs 65 us) stay on the
// non-persistent kernels.
template <bool INT8B, int AMODE>
inline bool persist_gemm_fits(const GemmParams &p) {
  if constexpr (INT8B || (AMODE != kAPlain && AMODE != kAConvVec)) {
    return false;
  } else {
    return dma_gemm_ok<false, AMODE>(p) && p.N % 128 == 0 && p.N <= kPersistMaxN && p.K >= 128 &&
           (p.K <= 512 || (p.K <= 1024 && p.N <= 1024)) &&
           2 * tiles_of(p, 128, 128) >= 3 * static_cast<int64_t>(device_cu_count()) && p.ldc % 8 == 0 &&
           (reinterpret_cast<uintptr_t>(p.C) & 15) == 0 && static_cast<int64_t>(p.M) * p.ldc * 2 < 0x7fffffff;
  }
}

template <int AMODE>
inline void launch_persist_default(const GemmParams &p, hipStream_t s) {
  launch_persist_gemm<128, 128, 4, 2, AMODE>(p, s);
}

}  // namespace teeny
