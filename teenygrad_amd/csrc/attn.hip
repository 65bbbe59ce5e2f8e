// Scaled-dot-product attention forward (flash / online softmax).
//
// Reference: flash_attention2_forward, kernels/teeny-kernels/src/nn/attention/
// flash_attn2.rs:52-158 — layout [BH, N, D] row-major (:18-21), one program
// per (q_row, bh), sequential online-softmax over every key row (:98-131),
// o = acc / l and L = m + log(l) (:133-157).  Non-causal only in the
// reference; `causal` here masks key j > query i (top-left aligned).
//
// Two kernels:
//
// fa_fwd_bf16 (the MI355X path).  One workgroup = 4 waves = 128 queries of
// one (b, h); each wave owns 32 queries.  K and V tiles of 64 keys are
// staged in LDS (double-buffered, next tile prefetched into registers while
// the current one is consumed).  Scores are computed transposed,
// S^T = K * Q^T, with v_mfma_f32_32x32x16_bf16: Q^T is the B operand and
// stays in registers for the whole key loop, and each lane's accumulator
// column is one query, so the softmax max/sum over keys is an in-lane
// reduction plus one exchange with lane ^ 32.  The probabilities are
// rounded to bf16 and fed, in exactly the registers the score MFMA wrote
// them to, as the B operand of O^T += V^T * P^T; V is written to LDS
// transposed ([d][key]) so that the matching A operand is two 8-byte LDS
// reads per MFMA.  Softmax runs in the exp2 domain (scale * log2 e folded
// into one multiply), fp32 throughout; the output is normalised once at the
// end.  Causal tiles beyond a wave's last query are skipped per wave and
// the query-block order is reversed so the heaviest blocks start first;
// workgroups of one (b, h) share an XCD (blockIdx.x = bh, 8 XCDs
// round-robin over the linear workgroup id) so K/V hit that XCD's L2.
//
// fa_fwd_f32 (fp32, any power-of-two head_dim <= 256).  The reference's
// per-query-row structure — grid (N_q, BH), one wave per query row — with
// the key loop vectorised across lanes: each lane scores one key of a
// 64-key chunk, and the chunk is folded into the running (m, l, acc) state.
#include "mfma.hpp"

namespace teeny {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

template <int D, bool CAUSAL>
__global__ __launch_bounds__(256, 2) void fa_fwd_bf16(const bf16 *__restrict__ Q,
                                                      const bf16 *__restrict__ K,
                                                      const bf16 *__restrict__ V,
                                                      bf16 *__restrict__ O, float *__restrict__ L,
                                                      int nq, int nk, float scale_log2, int nqb) {
  constexpr int BM = 128;          // queries per workgroup
  constexpr int BN = 64;           // keys per tile
  constexpr int KP = D + 8;        // K tile row pitch (elements): conflict-free 16-byte reads
  constexpr int VP = BN + 4;       // V^T tile row pitch (elements): conflict-free 8-byte reads
  constexpr int K_ELEMS = BN * KP;
  constexpr int V_ELEMS = D * VP;
  constexpr int STAGE = K_ELEMS + V_ELEMS;
  constexpr int CPR = D / 8;       // 16-byte chunks per row
  constexpr int RPP = 256 / CPR;   // K rows per load pass
  constexpr int KPASS = BN / RPP;  // K load passes
  constexpr int NS = D / 16;       // k-steps of the score MFMA
  constexpr int ND = D / 32;       // d-blocks of the output
  __shared__ __attribute__((aligned(16))) bf16 smem[2 * STAGE];

  const int bh = blockIdx.x;
  const int qb = nqb - 1 - static_cast<int>(blockIdx.y);
  const int tid = threadIdx.x;
  const int w = tid >> 6, lane = tid & 63, g = lane >> 5, c = lane & 31;
  const int q0 = qb * BM + w * 32;
  const int qi = q0 + c;

  const bf16 *Qb = Q + static_cast<int64_t>(bh) * nq * D;
  const bf16 *Kb = K + static_cast<int64_t>(bh) * nk * D;
  const bf16 *Vb = V + static_cast<int64_t>(bh) * nk * D;

  bf16x8 qf[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    if (qi < nq) {
      qf[s] = *reinterpret_cast<const bf16x8 *>(Qb + static_cast<int64_t>(qi) * D + 16 * s + 8 * g);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) qf[s][j] = static_cast<bf16>(0.0f);
    }
  }

  f32x16 acc[ND];
#pragma unroll
  for (int d = 0; d < ND; ++d) acc[d] = zero16();
  float m_run = -INFINITY, l_run = 0.0f;

  const int kv_end = CAUSAL ? min(nk, qb * BM + BM) : nk;
  const int n_tiles = (kv_end + BN - 1) / BN;
  const int wave_end = CAUSAL ? min(kv_end, q0 + 32) : kv_end;

  u32x4 kreg[KPASS];
  u32x4 vreg[4];
  const bool v_loader = tid < 16 * CPR;
  const int v_kq = tid / CPR, v_dc = tid % CPR;

  auto load_tile = [&](int kt) {
    const int kbase = kt * BN;
#pragma unroll
    for (int p = 0; p < KPASS; ++p) {
      const int row = tid / CPR + RPP * p;
      const int key = kbase + row;
      if (key < nk) {
        kreg[p] = *reinterpret_cast<const u32x4 *>(Kb + static_cast<int64_t>(key) * D + (tid % CPR) * 8);
      } else {
        kreg[p] = u32x4{0u, 0u, 0u, 0u};
      }
    }
    if (v_loader) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = kbase + 4 * v_kq + r;
        if (key < nk) {
          vreg[r] = *reinterpret_cast<const u32x4 *>(Vb + static_cast<int64_t>(key) * D + v_dc * 8);
        } else {
          vreg[r] = u32x4{0u, 0u, 0u, 0u};
        }
      }
    }
  };

  auto store_tile = [&](int buf) {
    bf16 *ks = smem + buf * STAGE;
    bf16 *vs = ks + K_ELEMS;
#pragma unroll
    for (int p = 0; p < KPASS; ++p) {
      const int row = tid / CPR + RPP * p;
      *reinterpret_cast<u32x4 *>(ks + row * KP + (tid % CPR) * 8) = kreg[p];
    }
    if (v_loader) {
      // vreg[r] holds V[key 4kq + r][8 dc .. 8 dc + 7]; write V^T[8 dc + i][4 kq .. 4 kq + 3].
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int wi = i >> 1;
        uint32_t lo, hi;
        if (i & 1) {
          lo = pack_hi(vreg[0][wi], vreg[1][wi]);
          hi = pack_hi(vreg[2][wi], vreg[3][wi]);
        } else {
          lo = pack_lo(vreg[0][wi], vreg[1][wi]);
          hi = pack_lo(vreg[2][wi], vreg[3][wi]);
        }
        uint2 pk;
        pk.x = lo;
        pk.y = hi;
        *reinterpret_cast<uint2 *>(vs + (v_dc * 8 + i) * VP + 4 * v_kq) = pk;
      }
    }
  };

  load_tile(0);
  store_tile(0);
  __syncthreads();

  for (int kt = 0; kt < n_tiles; ++kt) {
    if (kt + 1 < n_tiles) load_tile(kt + 1);
    const bf16 *ks = smem + (kt & 1) * STAGE;
    const bf16 *vs = ks + K_ELEMS;
    const int kbase = kt * BN;

    if (kbase < wave_end) {
      f32x16 sacc[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        sacc[kb] = zero16();
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          const bf16x8 a = *reinterpret_cast<const bf16x8 *>(ks + (kb * 32 + c) * KP + 16 * s + 8 * g);
          sacc[kb] = mfma32x32x16(a, qf[s], sacc[kb]);
        }
      }

      float t[2][16];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int v = 0; v < 16; ++v) t[kb][v] = sacc[kb][v] * scale_log2;

      const bool need_mask = (kbase + BN > nk) || (CAUSAL && kbase + BN - 1 > q0);
      if (need_mask) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int key = kbase + kb * 32 + mfma32_row(v, g);
            if (key >= nk || (CAUSAL && key > qi)) t[kb][v] = -INFINITY;
          }
      }

      float mx = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int v = 0; v < 16; ++v) mx = fmaxf(mx, t[kb][v]);
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float m_new = fmaxf(m_run, mx);
      const float m_use = m_new == -INFINITY ? 0.0f : m_new;
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);

      float psum = 0.0f;
      bf16x8 pf[2][2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const float p = __builtin_amdgcn_exp2f(t[kb][v] - m_use);
          psum += p;
          pf[kb][v >> 3][v & 7] = static_cast<bf16>(p);
        }
      l_run = l_run * alpha + psum;
      m_run = m_new;

#pragma unroll
      for (int d = 0; d < ND; ++d)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[d][v] *= alpha;

#pragma unroll
      for (int d = 0; d < ND; ++d) {
        const bf16 *vrow = vs + (d * 32 + c) * VP;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int tt = 0; tt < 2; ++tt) {
            const int col = kb * 32 + 16 * tt + 4 * g;
            const bf16x4 lo = *reinterpret_cast<const bf16x4 *>(vrow + col);
            const bf16x4 hi = *reinterpret_cast<const bf16x4 *>(vrow + col + 8);
            acc[d] = mfma32x32x16(cat8(lo, hi), pf[kb][tt], acc[d]);
          }
      }
    }

    if (kt + 1 < n_tiles) store_tile((kt + 1) & 1);
    __syncthreads();
  }

  const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
  if (qi < nq) {
    const float inv = 1.0f / l_tot;
    bf16 *orow = O + (static_cast<int64_t>(bh) * nq + qi) * D;
#pragma unroll
    for (int d = 0; d < ND; ++d)
#pragma unroll
      for (int v4 = 0; v4 < 4; ++v4) {
        bf16x4 o4;
#pragma unroll
        for (int i = 0; i < 4; ++i) o4[i] = static_cast<bf16>(acc[d][4 * v4 + i] * inv);
        *reinterpret_cast<bf16x4 *>(orow + d * 32 + 8 * v4 + 4 * g) = o4;
      }
    if (L != nullptr && g == 0) L[static_cast<int64_t>(bh) * nq + qi] = (m_run + log2f(l_tot)) * kLn2;
  }
}

// fp32 path: grid (nq, BH), one wave per query row (flash_attn2.rs:48-51).
template <int D>
__global__ __launch_bounds__(64) void fa_fwd_f32(const float *__restrict__ Q,
                                                 const float *__restrict__ K,
                                                 const float *__restrict__ V,
                                                 float *__restrict__ O, float *__restrict__ L,
                                                 int nq, int nk, float scale, int causal) {
  constexpr int DPL = (D + 63) / 64;  // output elements per lane
  __shared__ float qs[D];
  __shared__ float ps[64];
  const int qi = blockIdx.x;
  const int64_t bh = blockIdx.y;
  const int lane = threadIdx.x;
  const float *qrow = Q + (bh * nq + qi) * D;
  const float *Kb = K + bh * nk * D;
  const float *Vb = V + bh * nk * D;
  for (int d = lane; d < D; d += 64) qs[d] = qrow[d];
  __syncthreads();

  float acc[DPL];
#pragma unroll
  for (int i = 0; i < DPL; ++i) acc[i] = 0.0f;
  float m_i = -INFINITY, l_i = 0.0f;
  const int kend = causal ? min(nk, qi + 1) : nk;
  for (int k0 = 0; k0 < kend; k0 += 64) {
    const int key = k0 + lane;
    float s = -INFINITY;
    if (key < kend) {
      const float *krow = Kb + static_cast<int64_t>(key) * D;
      float dot = 0.0f;
#pragma unroll 8
      for (int d = 0; d < D; ++d) dot += qs[d] * krow[d];
      s = dot * scale;
    }
    const float m_new = fmaxf(m_i, wave_max(s));
    const float ed = expf(m_i - m_new);
    const float p = key < kend ? expf(s - m_new) : 0.0f;
    l_i = ed * l_i + wave_sum(p);
    ps[lane] = p;
    __syncthreads();
    const int cnt = min(64, kend - k0);
#pragma unroll
    for (int i = 0; i < DPL; ++i) {
      const int d = lane + 64 * i;
      if (d < D) {
        float a = ed * acc[i];
        for (int j = 0; j < cnt; ++j) a += ps[j] * Vb[static_cast<int64_t>(k0 + j) * D + d];
        acc[i] = a;
      }
    }
    m_i = m_new;
    __syncthreads();
  }
  float *orow = O + (bh * nq + qi) * D;
#pragma unroll
  for (int i = 0; i < DPL; ++i) {
    const int d = lane + 64 * i;
    if (d < D) orow[d] = acc[i] / l_i;
  }
  if (L != nullptr && lane == 0) L[bh * nq + qi] = m_i + logf(l_i);
}

template <int D>
static void launch_f32(const void *q, const void *k, const void *v, void *o, float *l, int nq,
                       int nk, float scale, int BH, int causal, hipStream_t s) {
  hipLaunchKernelGGL((fa_fwd_f32<D>), dim3(nq, BH), dim3(64), 0, s, static_cast<const float *>(q),
                     static_cast<const float *>(k), static_cast<const float *>(v),
                     static_cast<float *>(o), l, nq, nk, scale, causal);
}

template <int D>
static void launch_bf16(const void *q, const void *k, const void *v, void *o, float *l, int nq,
                        int nk, float scale, int BH, int causal, hipStream_t s) {
  const int nqb = (nq + 127) / 128;
  const float scale_log2 = scale * kLog2e;
  const dim3 grid(BH, nqb);
  if (causal) {
    hipLaunchKernelGGL((fa_fwd_bf16<D, true>), grid, dim3(256), 0, s,
                       static_cast<const bf16 *>(q), static_cast<const bf16 *>(k),
                       static_cast<const bf16 *>(v), static_cast<bf16 *>(o), l, nq, nk, scale_log2,
                       nqb);
  } else {
    hipLaunchKernelGGL((fa_fwd_bf16<D, false>), grid, dim3(256), 0, s,
                       static_cast<const bf16 *>(q), static_cast<const bf16 *>(k),
                       static_cast<const bf16 *>(v), static_cast<bf16 *>(o), l, nq, nk, scale_log2,
                       nqb);
  }
}

}  // namespace teeny

using namespace teeny;

extern "C" teeny_status teeny_flash_attention2_forward(const void *q, const void *k, const void *v,
                                                       void *o, float *l, int64_t n_ctx_q,
                                                       int64_t n_ctx_k, float softmax_scale,
                                                       int64_t BH, int64_t head_dim,
                                                       int32_t causal, teeny_dtype dtype,
                                                       teeny_stream stream) {
  const char *name = "flash_attention2_forward";
  TEENY_REQUIRE(n_ctx_q >= 0 && n_ctx_k >= 0 && BH >= 0, TEENY_ERR_SHAPE_MISMATCH,
                "flash_attention2_forward: negative size");
  if (n_ctx_q == 0 || BH == 0) return TEENY_OK;
  TEENY_REQUIRE(n_ctx_k > 0, TEENY_ERR_SHAPE_MISMATCH,
                "flash_attention2_forward: n_ctx_k must be positive (softmax over no keys)");
  TEENY_REQUIRE(n_ctx_q <= 0x7fffffff && n_ctx_k <= 0x7fffffff && BH <= 65535,
                TEENY_ERR_SHAPE_MISMATCH, "flash_attention2_forward: size out of range");
  TEENY_REQUIRE(q != nullptr && k != nullptr && v != nullptr && o != nullptr,
                TEENY_ERR_NULL_POINTER, "flash_attention2_forward: q/k/v/o");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int nq = static_cast<int>(n_ctx_q), nk = static_cast<int>(n_ctx_k);
  const int bh = static_cast<int>(BH);
  if (dtype == TEENY_F32) {
    TEENY_REQUIRE(n_ctx_q <= 0x7fffffff && BH <= 65535, TEENY_ERR_SHAPE_MISMATCH,
                  "flash_attention2_forward: grid out of range");
    switch (head_dim) {
      case 16: launch_f32<16>(q, k, v, o, l, nq, nk, softmax_scale, bh, causal, s); break;
      case 32: launch_f32<32>(q, k, v, o, l, nq, nk, softmax_scale, bh, causal, s); break;
      case 64: launch_f32<64>(q, k, v, o, l, nq, nk, softmax_scale, bh, causal, s); break;
      case 128: launch_f32<128>(q, k, v, o, l, nq, nk, softmax_scale, bh, causal, s); break;
      case 256: launch_f32<256>(q, k, v, o, l, nq, nk, softmax_scale, bh, causal, s); break;
      default:
        return fail(TEENY_ERR_UNSUPPORTED,
                    "flash_attention2_forward: f32 head_dim must be 16, 32, 64, 128 or 256");
    }
    return after_launch(name, s);
  }
  if (dtype == TEENY_BF16) {
    TEENY_REQUIRE(aligned(q, 16) && aligned(k, 16) && aligned(v, 16) && aligned(o, 16),
                  TEENY_ERR_MISALIGNED, "flash_attention2_forward: bf16 q/k/v/o must be 16-byte aligned");
    switch (head_dim) {
      case 64: launch_bf16<64>(q, k, v, o, l, nq, nk, softmax_scale, bh, causal, s); break;
      case 128: launch_bf16<128>(q, k, v, o, l, nq, nk, softmax_scale, bh, causal, s); break;
      default:
        return fail(TEENY_ERR_UNSUPPORTED,
                    "flash_attention2_forward: bf16 head_dim must be 64 or 128");
    }
    return after_launch(name, s);
  }
  return fail(TEENY_ERR_UNSUPPORTED_DTYPE, "flash_attention2_forward: dtype must be F32 or BF16");
}
