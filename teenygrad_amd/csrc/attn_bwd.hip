// Scaled-dot-product attention backward (flash attention 2).
//
// Reference: flash_attention2_backward_dq and flash_attention2_backward_dkv,
// kernels/teeny-kernels/src/nn/attention/flash_attn2.rs:173-447, layout
// [BH, N, D] row-major:
//   D_m  = sum_d O[m,d] dO[m,d]                       (per query row)
//   p_mn = exp(scale * Q_m . K_n - L_m)                (recomputed attention)
//   dS_mn = p_mn (dO_m . V_n - D_m)
//   dQ_m = scale * sum_n dS_mn K_n,  dK_n = scale * sum_m dS_mn Q_m,
//   dV_n = sum_m p_mn dO_m
// The reference runs one program per query row (dq, grid (N_q, BH)) and one
// per key row (dkv, grid (N_k, BH)), so neither needs atomics; the same
// split is kept here (deterministic, no atomics).  `causal` masks key n from
// query m when n > m (top-left aligned, as the forward).  Grouped K/V heads:
// query head h reads K/V head h / kv_group, and dK/dV of a K/V head sum over
// its kv_group query heads.
//
// bf16, head_dim 64 or 128 (the MI355X path): v_mfma_f32_32x32x16_bf16 with
// the operand orientation chosen so that every product's result feeds the
// next MFMA from the registers it was written to:
//   dkv: a wave owns 32 keys (columns of every 32x32 block), K^T and V^T
//        stay in registers as B operands; per 32-query block
//          S = Q K^T, dP = dO V^T            (A = Q / dO rows from LDS)
//          dV^T += dO^T P,  dK^T += Q^T dS   (A = dO^T / Q^T through
//                                             ds_read_b64_tr_b16; B = P, dS
//                                             rounded to bf16 in place)
//        Q and dO tiles of 64 queries are double-buffered in LDS by LDS-DMA.
//   dq:  a wave owns 32 queries; Q^T and dO^T are B operands in registers;
//        per 32-key block S^T = K Q^T, dP^T = V dO^T, dQ^T += K^T dS^T, with
//        K and V tiles of 64 keys double-buffered in LDS.
// D_m comes from a pre-pass over O and dO (the dq kernel also computes it
// in its own registers).  Every tile lives in LDS with an XOR swizzle of its
// 16-byte chunks chosen so that both the row reads (16 rows of one chunk)
// and the transposing reads (4 rows x 64 bytes per half-wave) touch
// distinct banks.
//
// Any other case (fp32, other head sizes, unaligned bf16): the reference's
// per-row structure, one wave per query row (dq) or key row (dkv), with the
// inner loop vectorised across lanes.
#include "mfma.hpp"

namespace teeny {

constexpr float kBwdLog2e = 1.4426950408889634f;

// ── generic kernels ───────────────────────────────────────────────────────

template <typename T, int D>
__global__ __launch_bounds__(64) void fa_bwd_dq_rows(const T *__restrict__ Q, const T *__restrict__ K,
                                                     const T *__restrict__ V, const T *__restrict__ O,
                                                     const T *__restrict__ dO, const float *__restrict__ L,
                                                     T *__restrict__ dQ, int nq, int nk, float scale, int causal,
                                                     int kv_group) {
  constexpr int DPL = (D + 63) / 64;
  __shared__ float qs[D], dos[D], dss[64];
  const int qi = blockIdx.x, lane = threadIdx.x;
  const int64_t bh = blockIdx.y;
  const int64_t row = bh * nq + qi;
  float dpart = 0.0f;
  for (int d = lane; d < D; d += 64) {
    const float g = to_f32(dO[row * D + d]);
    qs[d] = to_f32(Q[row * D + d]);
    dos[d] = g;
    dpart += to_f32(O[row * D + d]) * g;
  }
  const float delta = wave_sum(dpart);
  const float lq = L[row];
  __syncthreads();
  const T *Kb = K + (bh / kv_group) * nk * D;
  const T *Vb = V + (bh / kv_group) * nk * D;
  float acc[DPL];
#pragma unroll
  for (int i = 0; i < DPL; ++i) acc[i] = 0.0f;
  const int kend = causal ? min(nk, qi + 1) : nk;
  for (int k0 = 0; k0 < kend; k0 += 64) {
    const int key = k0 + lane;
    float ds = 0.0f;
    if (key < kend) {
      const T *kr = Kb + static_cast<int64_t>(key) * D;
      const T *vr = Vb + static_cast<int64_t>(key) * D;
      float s = 0.0f, dp = 0.0f;
#pragma unroll 8
      for (int d = 0; d < D; ++d) {
        s += qs[d] * to_f32(kr[d]);
        dp += dos[d] * to_f32(vr[d]);
      }
      ds = expf(s * scale - lq) * (dp - delta);
    }
    dss[lane] = ds;
    __syncthreads();
    const int cnt = min(64, kend - k0);
#pragma unroll
    for (int i = 0; i < DPL; ++i) {
      const int d = lane + 64 * i;
      if (d < D) {
        float a = acc[i];
        for (int j = 0; j < cnt; ++j) a += dss[j] * to_f32(Kb[static_cast<int64_t>(k0 + j) * D + d]);
        acc[i] = a;
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < DPL; ++i) {
    const int d = lane + 64 * i;
    if (d < D) dQ[row * D + d] = from_f32<T>(acc[i] * scale);
  }
}

// One wave per key row of K/V head blockIdx.y; `delta` (fp32 [BH, nq]) may be
// NULL, then D_m is recomputed from O and dO for every (key, query) pair.
template <typename T, int D>
__global__ __launch_bounds__(64) void fa_bwd_dkv_rows(const T *__restrict__ Q, const T *__restrict__ K,
                                                      const T *__restrict__ V, const T *__restrict__ O,
                                                      const T *__restrict__ dO, const float *__restrict__ L,
                                                      const float *__restrict__ delta, T *__restrict__ dK,
                                                      T *__restrict__ dV, int nq, int nk, float scale, int causal,
                                                      int kv_group) {
  constexpr int DPL = (D + 63) / 64;
  __shared__ float ks[D], vs[D], ps[64], dss[64];
  const int key = blockIdx.x, lane = threadIdx.x;
  const int64_t bhk = blockIdx.y;
  const int64_t krow = bhk * nk + key;
  for (int d = lane; d < D; d += 64) {
    ks[d] = to_f32(K[krow * D + d]);
    vs[d] = to_f32(V[krow * D + d]);
  }
  __syncthreads();
  float dk[DPL], dv[DPL];
#pragma unroll
  for (int i = 0; i < DPL; ++i) dk[i] = dv[i] = 0.0f;
  const int qstart = causal ? key : 0;
  for (int hq = 0; hq < kv_group; ++hq) {
    const int64_t bh = bhk * kv_group + hq;
    for (int q0 = qstart; q0 < nq; q0 += 64) {
      const int qi = q0 + lane;
      float p = 0.0f, ds = 0.0f;
      if (qi < nq) {
        const int64_t r = bh * nq + qi;
        float s = 0.0f, dp = 0.0f, dl = 0.0f;
#pragma unroll 8
        for (int d = 0; d < D; ++d) {
          const float g = to_f32(dO[r * D + d]);
          s += to_f32(Q[r * D + d]) * ks[d];
          dp += g * vs[d];
          if (delta == nullptr) dl += to_f32(O[r * D + d]) * g;
        }
        p = expf(s * scale - L[r]);
        ds = p * (dp - (delta != nullptr ? delta[r] : dl));
      }
      ps[lane] = p;
      dss[lane] = ds;
      __syncthreads();
      const int cnt = min(64, nq - q0);
#pragma unroll
      for (int i = 0; i < DPL; ++i) {
        const int d = lane + 64 * i;
        if (d < D) {
          float av = dv[i], ak = dk[i];
          for (int j = 0; j < cnt; ++j) {
            const int64_t r = (bh * nq + q0 + j) * D + d;
            av += ps[j] * to_f32(dO[r]);
            ak += dss[j] * to_f32(Q[r]);
          }
          dv[i] = av;
          dk[i] = ak;
        }
      }
      __syncthreads();
    }
  }
#pragma unroll
  for (int i = 0; i < DPL; ++i) {
    const int d = lane + 64 * i;
    if (d < D) {
      dK[krow * D + d] = from_f32<T>(dk[i] * scale);
      dV[krow * D + d] = from_f32<T>(dv[i]);
    }
  }
}

// ── bf16 MFMA kernels ───────────────────────────────────────────────────────

// Rows [row0, row0 + R) of an [n, D] bf16 matrix (buffer resource over its n
// rows: rows past n read as zeros) into a swizzled LDS tile, by LDS-DMA.
// Slot u = NT i + tid of the tile is row u / (D/8), chunk position u % (D/8).
template <int D, int R, int NT>
__device__ __forceinline__ void dma_tile(__amdgpu_buffer_rsrc_t rs, bf16 *dst, int row0, int tid) {
  constexpr int CPR = D / 8, RPI = NT / CPR, NLD = R * CPR / NT;
  static_assert(NLD >= 1 && R * CPR % NT == 0 && RPI % 16 == 0, "tile / thread shape");
  const int w = tid >> 6, lrow = tid / CPR, pos = tid % CPR;
  const int off = 2 * (lrow * D + ((pos ^ bswz<D>(lrow)) << 3));
#pragma unroll
  for (int i = 0; i < NLD; ++i)
    buffer_lds_dma16(rs, off + 2 * (row0 + RPI * i) * D,
                     __builtin_amdgcn_readfirstlane(lds_address(dst + (NT * i + 64 * w) * 8)));
}

// A operand from tile rows rb .. rb + 31 (rb a multiple of 32), k-step st:
// lane (g, r) holds row rb + r, elements 16 st + 8 g .. + 7.
template <int D>
__device__ __forceinline__ bf16x8 frag_row(const bf16 *tile, int rb, int st, int lane) {
  const int r = lane & 31, g = lane >> 5;
  return *reinterpret_cast<const bf16x8 *>(tile + (rb + r) * D + (((2 * st + g) ^ bswz<D>(r)) << 3));
}

// Registers 8t .. 8t+7 of a 32x32 fp32 result, rounded to bf16, as the B
// operand of a product whose k index runs over the result's rows.
__device__ __forceinline__ bf16x8 pack_b(const float *x, int t) {
  bf16x8 r;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const bf16x2 pr = cvt_pk_bf16(x[8 * t + 2 * j], x[8 * t + 2 * j + 1]);
    r[2 * j] = pr[0];
    r[2 * j + 1] = pr[1];
  }
  return r;
}

__device__ __forceinline__ bf16x8 load8(const bf16 *p) {
  const u32x4 raw = *reinterpret_cast<const u32x4 *>(p);
  bf16x8 v;
  __builtin_memcpy(&v, &raw, 16);
  return v;
}

__device__ __forceinline__ bf16x8 zero8() {
  const u32x4 z = {0u, 0u, 0u, 0u};
  bf16x8 v;
  __builtin_memcpy(&v, &z, 16);
  return v;
}

// Stores a C-layout result (rows d, column = this lane's row of `out`) times
// `mul` as bf16: lane (g, c) writes out[row][32 db + 8 a + 4 g + e].
template <int ND>
__device__ __forceinline__ void store_rows(bf16 *rowp, const f32x16 (&acc)[ND], float mul, int g) {
#pragma unroll
  for (int db = 0; db < ND; ++db)
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      bf16x4 o4;
#pragma unroll
      for (int e = 0; e < 4; ++e) o4[e] = static_cast<bf16>(acc[db][4 * a + e] * mul);
      *reinterpret_cast<bf16x4 *>(rowp + 32 * db + 8 * a + 4 * g) = o4;
    }
}

// D_m = sum_d O[m, d] dO[m, d] in fp32: D/8 lanes per row, 16 bytes each.
template <int D>
__global__ __launch_bounds__(256) void fa_bwd_delta_bf16(const bf16 *__restrict__ O, const bf16 *__restrict__ dO,
                                                         float *__restrict__ delta, int64_t rows) {
  constexpr int CPR = D / 8;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t row = t / CPR;
  float s = 0.0f;
  if (row < rows) {
    const bf16x8 o = load8(O + t * 8), g = load8(dO + t * 8);
#pragma unroll
    for (int j = 0; j < 8; ++j) s += static_cast<float>(o[j]) * static_cast<float>(g[j]);
  }
#pragma unroll
  for (int off = CPR / 2; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
  if (row < rows && t % CPR == 0) delta[row] = s;
}

// dK, dV for the 32 * WAVES keys of one workgroup (wave w: keys k0 + 0..31),
// head_dim 64.  (At head_dim 128 the K^T / V^T operands and both
// accumulators take 192 of a lane's registers: one workgroup per CU; that
// size runs fa_bwd_dkv_vl_bf16 below, 923 -> 790 us at B*H = 256, S = 2048
// causal.)
template <int D, bool CAUSAL, int WAVES>
__global__ __launch_bounds__(64 * WAVES, (D == 128 ? 4 : 8) / WAVES) void fa_bwd_dkv_bf16(
    const bf16 *__restrict__ Q, const bf16 *__restrict__ K, const bf16 *__restrict__ V,
    const bf16 *__restrict__ dO, const float *__restrict__ L, const float *__restrict__ Delta,
    bf16 *__restrict__ dK, bf16 *__restrict__ dV, int nq, int nk, float scale, float sc, int nkb, int kv_group) {
  constexpr int NT = 64 * WAVES, BN = 32 * WAVES, BM = 64, NS = D / 16, ND = D / 32, TILE = BM * D;
  __shared__ __attribute__((aligned(16))) bf16 qbuf[2][TILE], dobuf[2][TILE];
  __shared__ __attribute__((aligned(16))) float lbuf[2][BM], dbuf[2][BM];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, c = lane & 31;
  const int tile_id = xcd_remap(blockIdx.x, gridDim.x);
  const int bhk = tile_id / nkb, kblk = tile_id % nkb;
  const int kb0 = kblk * BN, k0 = kb0 + 32 * w, key = k0 + c;
  const bf16 *Kr = K + (static_cast<int64_t>(bhk) * nk + key) * D;
  const bf16 *Vr = V + (static_cast<int64_t>(bhk) * nk + key) * D;
  bf16x8 kT[NS], vT[NS];
#pragma unroll
  for (int st = 0; st < NS; ++st) {
    kT[st] = key < nk ? load8(Kr + 16 * st + 8 * g) : zero8();
    vT[st] = key < nk ? load8(Vr + 16 * st + 8 * g) : zero8();
  }
  f32x16 dk[ND], dv[ND];
#pragma unroll
  for (int d = 0; d < ND; ++d) dk[d] = dv[d] = zero16();

  const int qt0 = CAUSAL ? kb0 / BM : 0;
  const int per_head = (nq + BM - 1) / BM - qt0;
  const int total = per_head > 0 ? per_head * kv_group : 0;
  float l_next = 0.0f, d_next = 0.0f;
  // starts the loads of tile idx (query head, query tile) into buffer b; the
  // L / D_m values of its rows wait in registers of the first BM threads
  auto issue = [&](int idx, int b) __attribute__((always_inline)) {
    const int hq = idx / per_head, qt = qt0 + idx % per_head;
    const int64_t bh = static_cast<int64_t>(bhk) * kv_group + hq;
    dma_tile<D, BM, NT>(buffer_rsrc(Q + bh * nq * D, nq * D * 2), qbuf[b], qt * BM, tid);
    dma_tile<D, BM, NT>(buffer_rsrc(dO + bh * nq * D, nq * D * 2), dobuf[b], qt * BM, tid);
    if (tid < BM) {
      const int row = qt * BM + tid;
      // rows past nq: L = +inf makes p = 0
      l_next = row < nq ? L[bh * nq + row] * kBwdLog2e : INFINITY;
      d_next = row < nq ? Delta[bh * nq + row] : 0.0f;
    }
  };
  if (total > 0) {
    issue(0, 0);
    if (tid < BM) {
      lbuf[0][tid] = l_next;
      dbuf[0][tid] = d_next;
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  }
  for (int idx = 0; idx < total; ++idx) {
    const int b = idx & 1;
    if (idx + 1 < total) issue(idx + 1, b ^ 1);
    const int qt = qt0 + idx % per_head;
    const bf16 *qs = qbuf[b], *dos = dobuf[b];
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      const int q0 = qt * BM + 32 * sb;
      if (q0 >= nq || (CAUSAL && q0 + 31 < k0)) continue;  // wave-uniform: no query of the block sees these keys
      f32x16 s = zero16(), dp = zero16();
#pragma unroll
      for (int st = 0; st < NS; ++st) {
        s = mfma32x32x16(frag_row<D>(qs, 32 * sb, st, lane), kT[st], s);
        dp = mfma32x32x16(frag_row<D>(dos, 32 * sb, st, lane), vT[st], dp);
      }
      float p[16], ds[16];
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const f32x4 l4 = *reinterpret_cast<const f32x4 *>(&lbuf[b][32 * sb + 8 * a + 4 * g]);
        const f32x4 d4 = *reinterpret_cast<const f32x4 *>(&dbuf[b][32 * sb + 8 * a + 4 * g]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int v = 4 * a + e;
          float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(s[v], sc, -l4[e]));
          if (CAUSAL && key > q0 + 8 * a + 4 * g + e) pv = 0.0f;
          p[v] = pv;
          ds[v] = pv * (dp[v] - d4[e]);
        }
      }
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const bf16x8 pb = pack_b(p, t), db8 = pack_b(ds, t);
#pragma unroll
        for (int d = 0; d < ND; ++d) {
          dv[d] = mfma32x32x16(frag_tr<D>(dos, 32 * sb + 16 * t, d, lane), pb, dv[d]);
          dk[d] = mfma32x32x16(frag_tr<D>(qs, 32 * sb + 16 * t, d, lane), db8, dk[d]);
        }
      }
    }
    if (idx + 1 < total && tid < BM) {
      lbuf[b ^ 1][tid] = l_next;
      dbuf[b ^ 1][tid] = d_next;
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  }
  if (key < nk) {
    const int64_t row = static_cast<int64_t>(bhk) * nk + key;
    store_rows<ND>(dK + row * D, dk, scale, g);
    store_rows<ND>(dV + row * D, dv, 1.0f, g);
  }
}

// dK, dV at head_dim 128 in two workgroups per CU: the same products as
// fa_bwd_dkv_bf16 for the 128 keys of a workgroup, with V^T read from an LDS
// copy of the workgroup's V rows instead of registers and query tiles of 32
// rows, so that a wave fits 256 registers (K^T 32, the dK / dV accumulators
// 128, S and dP 32) and each SIMD runs two waves, whose exponentials and
// MFMAs overlap.
template <bool CAUSAL>
__global__ __launch_bounds__(256, 2) void fa_bwd_dkv_vl_bf16(
    const bf16 *__restrict__ Q, const bf16 *__restrict__ K, const bf16 *__restrict__ V,
    const bf16 *__restrict__ dO, const float *__restrict__ L, const float *__restrict__ Delta,
    bf16 *__restrict__ dK, bf16 *__restrict__ dV, int nq, int nk, float scale, float sc, int nkb, int kv_group) {
  constexpr int D = 128, NT = 256, BN = 128, BM = 32, NS = D / 16, ND = D / 32, TILE = BM * D;
  __shared__ __attribute__((aligned(16))) bf16 qbuf[2][TILE], dobuf[2][TILE], vl[BN * D];
  __shared__ __attribute__((aligned(16))) float lbuf[2][BM], dbuf[2][BM];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, c = lane & 31;
  const int tile_id = xcd_remap(blockIdx.x, gridDim.x);
  const int bhk = tile_id / nkb, kblk = tile_id % nkb;
  const int kb0 = kblk * BN, k0 = kb0 + 32 * w, key = k0 + c;
  const bf16 *Kr = K + (static_cast<int64_t>(bhk) * nk + key) * D;
  // the workgroup's V rows (rows past nk read as zeros), one DMA pass
  dma_tile<D, BN, NT>(buffer_rsrc(V + static_cast<int64_t>(bhk) * nk * D, nk * D * 2), vl, kb0, tid);
  bf16x8 kT[NS];
#pragma unroll
  for (int st = 0; st < NS; ++st) kT[st] = key < nk ? load8(Kr + 16 * st + 8 * g) : zero8();
  f32x16 dk[ND], dv[ND];
#pragma unroll
  for (int d = 0; d < ND; ++d) dk[d] = dv[d] = zero16();

  const int qt0 = CAUSAL ? kb0 / BM : 0;
  const int per_head = (nq + BM - 1) / BM - qt0;
  const int total = per_head > 0 ? per_head * kv_group : 0;
  float l_next = 0.0f, d_next = 0.0f;
  auto issue = [&](int idx, int b) __attribute__((always_inline)) {
    const int hq = idx / per_head, qt = qt0 + idx % per_head;
    const int64_t bh = static_cast<int64_t>(bhk) * kv_group + hq;
    dma_tile<D, BM, NT>(buffer_rsrc(Q + bh * nq * D, nq * D * 2), qbuf[b], qt * BM, tid);
    dma_tile<D, BM, NT>(buffer_rsrc(dO + bh * nq * D, nq * D * 2), dobuf[b], qt * BM, tid);
    if (tid < BM) {
      const int row = qt * BM + tid;
      l_next = row < nq ? L[bh * nq + row] * kBwdLog2e : INFINITY;
      d_next = row < nq ? Delta[bh * nq + row] : 0.0f;
    }
  };
  if (total > 0) issue(0, 0);
  if (tid < BM) {
    lbuf[0][tid] = l_next;
    dbuf[0][tid] = d_next;
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  for (int idx = 0; idx < total; ++idx) {
    const int b = idx & 1;
    if (idx + 1 < total) issue(idx + 1, b ^ 1);
    const int q0 = (qt0 + idx % per_head) * BM;
    const bf16 *qs = qbuf[b], *dos = dobuf[b];
    // wave-uniform: skip when no query of the tile sees these keys
    if (q0 < nq && !(CAUSAL && q0 + BM - 1 < k0)) {
      f32x16 s = zero16(), dp = zero16();
      // wave priority 1 over S and dP, 0 over the exponentials and the dV /
      // dK products: of the two waves on a SIMD, the one starting a tile's
      // products issues first (1.350 -> 1.319 ms for the causal S = 2048
      // backward)
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int st = 0; st < NS; ++st) {
        s = mfma32x32x16(frag_row<D>(qs, 0, st, lane), kT[st], s);
        dp = mfma32x32x16(frag_row<D>(dos, 0, st, lane), frag_row<D>(vl, 32 * w, st, lane), dp);
      }
      __builtin_amdgcn_s_setprio(0);
      float p[16], ds[16];
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const f32x4 l4 = *reinterpret_cast<const f32x4 *>(&lbuf[b][8 * a + 4 * g]);
        const f32x4 d4 = *reinterpret_cast<const f32x4 *>(&dbuf[b][8 * a + 4 * g]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int v = 4 * a + e;
          float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(s[v], sc, -l4[e]));
          if (CAUSAL && key > q0 + 8 * a + 4 * g + e) pv = 0.0f;
          p[v] = pv;
          ds[v] = pv * (dp[v] - d4[e]);
        }
      }
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const bf16x8 pb = pack_b(p, t), db8 = pack_b(ds, t);
#pragma unroll
        for (int d = 0; d < ND; ++d) {
          dv[d] = mfma32x32x16(frag_tr<D>(dos, 16 * t, d, lane), pb, dv[d]);
          dk[d] = mfma32x32x16(frag_tr<D>(qs, 16 * t, d, lane), db8, dk[d]);
        }
      }
    }
    if (idx + 1 < total && tid < BM) {
      lbuf[b ^ 1][tid] = l_next;
      dbuf[b ^ 1][tid] = d_next;
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  }
  if (key < nk) {
    const int64_t row = static_cast<int64_t>(bhk) * nk + key;
    store_rows<ND>(dK + row * D, dk, scale, g);
    store_rows<ND>(dV + row * D, dv, 1.0f, g);
  }
}

// dQ for the 32 * WAVES queries of one workgroup (wave w: queries q0 + 0..31);
// also writes D_m to delta_out when that is not NULL.
template <int D, bool CAUSAL, int WAVES>
__global__ __launch_bounds__(64 * WAVES, 8 / WAVES) void fa_bwd_dq_bf16(
    const bf16 *__restrict__ Q, const bf16 *__restrict__ K, const bf16 *__restrict__ V,
    const bf16 *__restrict__ O, const bf16 *__restrict__ dO, const float *__restrict__ L, bf16 *__restrict__ dQ,
    float *__restrict__ delta_out, int nq, int nk, float scale, float sc, int nqb, int kv_group) {
  constexpr int NT = 64 * WAVES, BM = 32 * WAVES, BN = 64, NS = D / 16, ND = D / 32, TILE = BN * D;
  __shared__ __attribute__((aligned(16))) bf16 kbuf[2][TILE], vbuf[2][TILE];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, c = lane & 31;
  const int tile_id = xcd_remap(blockIdx.x, gridDim.x);
  const int bh = tile_id / nqb, slot = tile_id % nqb;
  const int qb = CAUSAL ? nqb - 1 - slot : slot;  // causal: heaviest blocks first
  const int q0 = qb * BM + 32 * w, qi = q0 + c;
  const int64_t qrow = static_cast<int64_t>(bh) * nq + qi;
  bf16x8 qT[NS], doT[NS];
  float dpart = 0.0f;
#pragma unroll
  for (int st = 0; st < NS; ++st) {
    if (qi < nq) {
      qT[st] = load8(Q + qrow * D + 16 * st + 8 * g);
      doT[st] = load8(dO + qrow * D + 16 * st + 8 * g);
      const bf16x8 o = load8(O + qrow * D + 16 * st + 8 * g);
#pragma unroll
      for (int j = 0; j < 8; ++j) dpart += static_cast<float>(o[j]) * static_cast<float>(doT[st][j]);
    } else {
      qT[st] = doT[st] = zero8();
    }
  }
  // the other half of the row's elements sits in lane ^ 32
  const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(dpart), __float_as_uint(dpart), false, false);
  const float delta = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
  const float l2 = qi < nq ? L[qrow] * kBwdLog2e : 0.0f;
  if (delta_out != nullptr && g == 0 && qi < nq) delta_out[qrow] = delta;

  f32x16 dq[ND];
#pragma unroll
  for (int d = 0; d < ND; ++d) dq[d] = zero16();
  const int kv_end = CAUSAL ? min(nk, qb * BM + BM) : nk;
  const int n_kt = (kv_end + BN - 1) / BN;
  const int wave_end = CAUSAL ? min(kv_end, q0 + 32) : kv_end;
  const bf16 *Kb = K + static_cast<int64_t>(bh / kv_group) * nk * D;
  const bf16 *Vb = V + static_cast<int64_t>(bh / kv_group) * nk * D;
  const __amdgpu_buffer_rsrc_t krs = buffer_rsrc(Kb, nk * D * 2), vrs = buffer_rsrc(Vb, nk * D * 2);
  if (n_kt > 0) {
    dma_tile<D, BN, NT>(krs, kbuf[0], 0, tid);
    dma_tile<D, BN, NT>(vrs, vbuf[0], 0, tid);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  }
  for (int kt = 0; kt < n_kt; ++kt) {
    const int b = kt & 1;
    if (kt + 1 < n_kt) {
      dma_tile<D, BN, NT>(krs, kbuf[b ^ 1], (kt + 1) * BN, tid);
      dma_tile<D, BN, NT>(vrs, vbuf[b ^ 1], (kt + 1) * BN, tid);
    }
    const bf16 *ks = kbuf[b], *vs = vbuf[b];
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      const int kbase = kt * BN + 32 * sb;
      if (kbase >= wave_end) continue;  // wave-uniform: past nk, or causal keys after the wave's last query
      f32x16 s = zero16(), dp = zero16();
#pragma unroll
      for (int st = 0; st < NS; ++st) {
        s = mfma32x32x16(frag_row<D>(ks, 32 * sb, st, lane), qT[st], s);
        dp = mfma32x32x16(frag_row<D>(vs, 32 * sb, st, lane), doT[st], dp);
      }
      float ds[16];
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int kv = kbase + mfma32_row(v, g);
        float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(s[v], sc, -l2));
        if (kv >= nk || (CAUSAL && kv > qi)) pv = 0.0f;
        ds[v] = pv * (dp[v] - delta);
      }
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const bf16x8 db8 = pack_b(ds, t);
#pragma unroll
        for (int d = 0; d < ND; ++d) dq[d] = mfma32x32x16(frag_tr<D>(ks, 32 * sb + 16 * t, d, lane), db8, dq[d]);
      }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  }
  if (qi < nq) store_rows<ND>(dQ + qrow * D, dq, scale, g);
}

__global__ __launch_bounds__(256) void fa_bwd_zero(uint32_t *__restrict__ p, int64_t words) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < words;
       i += static_cast<int64_t>(gridDim.x) * 256)
    p[i] = 0u;
}

// ── launchers ───────────────────────────────────────────────────────────────

constexpr int kBwdWaves = 4;

struct BwdArgs {
  const void *q, *k, *v, *o, *dout;
  const float *l;
  void *dq, *dk, *dv;
  int BH, nq, nk, D, causal, group;  // BH counts query heads; K/V heads = BH / group
  float scale;
  hipStream_t s;
};

template <typename T, int D>
static void rows_dq(const BwdArgs &a) {
  hipLaunchKernelGGL((fa_bwd_dq_rows<T, D>), dim3(a.nq, a.BH), dim3(64), 0, a.s, static_cast<const T *>(a.q),
                     static_cast<const T *>(a.k), static_cast<const T *>(a.v), static_cast<const T *>(a.o),
                     static_cast<const T *>(a.dout), a.l, static_cast<T *>(a.dq), a.nq, a.nk, a.scale, a.causal,
                     a.group);
}

template <typename T, int D>
static void rows_dkv(const BwdArgs &a, const float *delta) {
  hipLaunchKernelGGL((fa_bwd_dkv_rows<T, D>), dim3(a.nk, a.BH / a.group), dim3(64), 0, a.s,
                     static_cast<const T *>(a.q), static_cast<const T *>(a.k), static_cast<const T *>(a.v),
                     static_cast<const T *>(a.o), static_cast<const T *>(a.dout), a.l, delta,
                     static_cast<T *>(a.dk), static_cast<T *>(a.dv), a.nq, a.nk, a.scale, a.causal, a.group);
}

template <typename T>
static bool rows_launch(const BwdArgs &a, bool dq, const float *delta) {
#define TEENY_BWD_ROWS(DD)          \
  case DD:                          \
    if (dq) rows_dq<T, DD>(a);      \
    else rows_dkv<T, DD>(a, delta); \
    return true;
  switch (a.D) {
    TEENY_BWD_ROWS(16)
    TEENY_BWD_ROWS(32)
    TEENY_BWD_ROWS(64)
    TEENY_BWD_ROWS(128)
    TEENY_BWD_ROWS(256)
    default: return false;
  }
#undef TEENY_BWD_ROWS
}

template <int D>
static void mfma_delta(const BwdArgs &a, float *delta) {
  const int64_t rows = static_cast<int64_t>(a.BH) * a.nq;
  const int64_t threads = rows * (D / 8);
  hipLaunchKernelGGL((fa_bwd_delta_bf16<D>), dim3(static_cast<unsigned>(cdiv(threads, 256))), dim3(256), 0, a.s,
                     static_cast<const bf16 *>(a.o), static_cast<const bf16 *>(a.dout), delta, rows);
}

template <int D, bool CAUSAL>
static void mfma_dkv(const BwdArgs &a, const float *delta) {
  constexpr int BN = 32 * kBwdWaves;
  const int nkb = (a.nk + BN - 1) / BN;
  if constexpr (D == 128 && kBwdWaves == 4) {
    hipLaunchKernelGGL((fa_bwd_dkv_vl_bf16<CAUSAL>), dim3((a.BH / a.group) * nkb), dim3(256), 0, a.s,
                       static_cast<const bf16 *>(a.q), static_cast<const bf16 *>(a.k),
                       static_cast<const bf16 *>(a.v), static_cast<const bf16 *>(a.dout), a.l, delta,
                       static_cast<bf16 *>(a.dk), static_cast<bf16 *>(a.dv), a.nq, a.nk, a.scale,
                       a.scale * kBwdLog2e, nkb, a.group);
    return;
  }
  hipLaunchKernelGGL((fa_bwd_dkv_bf16<D, CAUSAL, kBwdWaves>), dim3((a.BH / a.group) * nkb), dim3(64 * kBwdWaves), 0,
                     a.s, static_cast<const bf16 *>(a.q), static_cast<const bf16 *>(a.k),
                     static_cast<const bf16 *>(a.v), static_cast<const bf16 *>(a.dout), a.l, delta,
                     static_cast<bf16 *>(a.dk), static_cast<bf16 *>(a.dv), a.nq, a.nk, a.scale, a.scale * kBwdLog2e,
                     nkb, a.group);
}

template <int D, bool CAUSAL>
static void mfma_dq(const BwdArgs &a, float *delta_out) {
  constexpr int BM = 32 * kBwdWaves;
  const int nqb = (a.nq + BM - 1) / BM;
  hipLaunchKernelGGL((fa_bwd_dq_bf16<D, CAUSAL, kBwdWaves>), dim3(a.BH * nqb), dim3(64 * kBwdWaves), 0, a.s,
                     static_cast<const bf16 *>(a.q), static_cast<const bf16 *>(a.k), static_cast<const bf16 *>(a.v),
                     static_cast<const bf16 *>(a.o), static_cast<const bf16 *>(a.dout), a.l,
                     static_cast<bf16 *>(a.dq), delta_out, a.nq, a.nk, a.scale, a.scale * kBwdLog2e, nqb, a.group);
}

template <int D>
static void mfma_run(const BwdArgs &a, int which, float *delta) {
  // which: 0 = delta pre-pass, 1 = dkv, 2 = dq (writes delta when not NULL)
  if (which == 0) mfma_delta<D>(a, delta);
  else if (which == 1) (a.causal ? mfma_dkv<D, true> : mfma_dkv<D, false>)(a, delta);
  else (a.causal ? mfma_dq<D, true> : mfma_dq<D, false>)(a, delta);
}

static void mfma_step(const BwdArgs &a, int which, float *delta) {
  if (a.D == 64) mfma_run<64>(a, which, delta);
  else mfma_run<128>(a, which, delta);
}

// The MFMA kernels apply: bf16, head_dim 64 / 128, 16-byte aligned tensors,
// and every head's Q / dO / K / V below 2 GiB (32-bit buffer offsets).
static bool mfma_ok(const BwdArgs &a, teeny_dtype dtype) {
  if (dtype != TEENY_BF16 || (a.D != 64 && a.D != 128)) return false;
  for (const void *p : {a.q, a.k, a.v, a.o, a.dout}) if (!aligned(p, 16)) return false;
  for (const void *p : {a.dq, a.dk, a.dv}) if (p != nullptr && !aligned(p, 16)) return false;
  const int64_t most = std::max<int64_t>(a.nq, a.nk) + 256;
  return most * a.D * 2 <= 0x7fffffff;
}

static size_t delta_bytes(const BwdArgs &a) { return static_cast<size_t>(a.BH) * a.nq * sizeof(float); }

// which: 1 dq only, 2 dk/dv only, 3 all three.
static teeny_status bwd_entry(BwdArgs a, int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t nq, int64_t nk,
                              int64_t D, int which, teeny_dtype dtype, const char *name) {
  const std::string nm(name);
  TEENY_REQUIRE(nq >= 0 && nk >= 0 && batch >= 0 && q_heads >= 0 && kv_heads >= 0, TEENY_ERR_SHAPE_MISMATCH,
                nm + ": negative size");
  TEENY_REQUIRE(kv_heads > 0 ? q_heads % kv_heads == 0 : q_heads == 0, TEENY_ERR_SHAPE_MISMATCH,
                nm + ": q_heads must be a multiple of kv_heads");
  TEENY_REQUIRE(dtype == TEENY_F32 || dtype == TEENY_BF16, TEENY_ERR_UNSUPPORTED_DTYPE,
                nm + ": dtype must be F32 or BF16");
  TEENY_REQUIRE(D == 16 || D == 32 || D == 64 || D == 128 || D == 256, TEENY_ERR_UNSUPPORTED,
                nm + ": head_dim must be 16, 32, 64, 128 or 256");
  const int64_t BH = batch * q_heads;
  if (BH == 0 || (nq == 0 && nk == 0)) return TEENY_OK;
  TEENY_REQUIRE(nq <= 0x7fffffff && nk <= 0x7fffffff && BH <= 65535 && BH * (nq + 127) / 128 <= 0x7fffffff &&
                    BH * (nk + 127) / 128 <= 0x7fffffff,
                TEENY_ERR_SHAPE_MISMATCH, nm + ": size out of range");
  TEENY_REQUIRE(a.q != nullptr && a.k != nullptr && a.v != nullptr && a.o != nullptr && a.dout != nullptr &&
                    a.l != nullptr,
                TEENY_ERR_NULL_POINTER, nm + ": q/k/v/o/do/l");
  TEENY_REQUIRE(!(which & 1) || a.dq != nullptr, TEENY_ERR_NULL_POINTER, nm + ": dq");
  TEENY_REQUIRE(!(which & 2) || (a.dk != nullptr && a.dv != nullptr), TEENY_ERR_NULL_POINTER, nm + ": dk/dv");
  a.BH = static_cast<int>(BH);
  a.nq = static_cast<int>(nq);
  a.nk = static_cast<int>(nk);
  a.D = static_cast<int>(D);
  a.group = static_cast<int>(q_heads / kv_heads);
  const size_t esz = dtype == TEENY_F32 ? 4 : 2;
  if (nq == 0) {  // no queries: dK = dV = 0 (a fill kernel, so the call may be graph-captured)
    if (which & 2) {
      const int64_t words = (BH / a.group) * nk * D * static_cast<int64_t>(esz) / 4;
      const unsigned blocks = static_cast<unsigned>(std::min<int64_t>(cdiv(words, 256), 65536));
      hipLaunchKernelGGL(fa_bwd_zero, dim3(blocks), dim3(256), 0, a.s, static_cast<uint32_t *>(a.dk), words);
      hipLaunchKernelGGL(fa_bwd_zero, dim3(blocks), dim3(256), 0, a.s, static_cast<uint32_t *>(a.dv), words);
    }
    return after_launch(name, a.s);
  }
  TEENY_REQUIRE(nk > 0, TEENY_ERR_SHAPE_MISMATCH, nm + ": n_ctx_k must be positive (softmax over no keys)");
  if (mfma_ok(a, dtype)) {
    const Scratch scr = stream_scratch(a.s);
    const bool ws = scr.ptr != nullptr && scr.bytes >= delta_bytes(a);
    if (which == 1) {
      mfma_step(a, 2, nullptr);
    } else if (which == 3) {
      if (ws) {  // dq first, writing D_m for the dk/dv kernel
        float *delta = static_cast<float *>(scr.ptr);
        mfma_step(a, 2, delta);
        mfma_step(a, 1, delta);
      } else {  // D_m parked in dq's memory until the dq kernel overwrites it
        float *delta = static_cast<float *>(a.dq);
        mfma_step(a, 0, delta);
        mfma_step(a, 1, delta);
        mfma_step(a, 2, nullptr);
      }
    } else if (ws) {
      float *delta = static_cast<float *>(scr.ptr);
      mfma_step(a, 0, delta);
      mfma_step(a, 1, delta);
    } else {
      rows_launch<bf16>(a, false, nullptr);
    }
    return after_launch(name, a.s);
  }
  if (which & 1) (dtype == TEENY_F32 ? rows_launch<float> : rows_launch<bf16>)(a, true, nullptr);
  if (which & 2) (dtype == TEENY_F32 ? rows_launch<float> : rows_launch<bf16>)(a, false, nullptr);
  return after_launch(name, a.s);
}

}  // namespace teeny

using namespace teeny;

extern "C" {

teeny_status teeny_flash_attention2_backward_dq(const void *q, const void *k, const void *v, const void *o,
                                                const void *dout, const float *l, void *dq, int64_t n_ctx_q,
                                                int64_t n_ctx_k, float softmax_scale, int64_t BH, int64_t head_dim,
                                                int32_t causal, teeny_dtype dtype, teeny_stream stream) {
  BwdArgs a{q, k, v, o, dout, l, dq, nullptr, nullptr, 0, 0, 0, 0, causal != 0, 1, softmax_scale,
            static_cast<hipStream_t>(stream)};
  return bwd_entry(a, BH, 1, 1, n_ctx_q, n_ctx_k, head_dim, 1, dtype, "flash_attention2_backward_dq");
}

teeny_status teeny_flash_attention2_backward_dkv(const void *q, const void *k, const void *v, const void *o,
                                                 const void *dout, const float *l, void *dk, void *dv,
                                                 int64_t n_ctx_q, int64_t n_ctx_k, float softmax_scale, int64_t BH,
                                                 int64_t head_dim, int32_t causal, teeny_dtype dtype,
                                                 teeny_stream stream) {
  BwdArgs a{q, k, v, o, dout, l, nullptr, dk, dv, 0, 0, 0, 0, causal != 0, 1, softmax_scale,
            static_cast<hipStream_t>(stream)};
  return bwd_entry(a, BH, 1, 1, n_ctx_q, n_ctx_k, head_dim, 2, dtype, "flash_attention2_backward_dkv");
}

teeny_status teeny_attention_backward(const void *q, const void *k, const void *v, const void *o, const void *dout,
                                      const float *l, void *dq, void *dk, void *dv, int64_t batch, int64_t q_heads,
                                      int64_t kv_heads, int64_t n_ctx_q, int64_t n_ctx_k, int64_t head_dim,
                                      float softmax_scale, int32_t causal, teeny_dtype dtype, teeny_stream stream) {
  BwdArgs a{q, k, v, o, dout, l, dq, dk, dv, 0, 0, 0, 0, causal != 0, 1, softmax_scale,
            static_cast<hipStream_t>(stream)};
  return bwd_entry(a, batch, q_heads, kv_heads, n_ctx_q, n_ctx_k, head_dim, 3, dtype, "attention_backward");
}

teeny_status teeny_attention_backward_workspace_size(int64_t batch, int64_t q_heads, int64_t n_ctx_q,
                                                     size_t *bytes) {
  TEENY_REQUIRE(bytes != nullptr, TEENY_ERR_NULL_POINTER, "attention_backward_workspace_size: bytes");
  *bytes = 0;
  TEENY_REQUIRE(batch >= 0 && q_heads >= 0 && n_ctx_q >= 0, TEENY_ERR_SHAPE_MISMATCH,
                "attention_backward_workspace_size: negative size");
  // the limits the backward itself enforces: B*H <= 65535 and n_ctx_q < 2^31,
  // so the product below is at most 2^47 and cannot overflow
  TEENY_REQUIRE(q_heads == 0 || batch <= 65535 / q_heads, TEENY_ERR_SHAPE_MISMATCH,
                "attention_backward_workspace_size: batch * q_heads exceeds 65535");
  TEENY_REQUIRE(n_ctx_q <= 0x7fffffff, TEENY_ERR_SHAPE_MISMATCH,
                "attention_backward_workspace_size: n_ctx_q exceeds 2^31 - 1");
  *bytes = static_cast<size_t>(batch * q_heads * n_ctx_q) * sizeof(float);
  return TEENY_OK;
}

}  // extern "C"
