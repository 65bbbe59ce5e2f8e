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
// fa_fwd_bf16 (the MI355X path).  One workgroup = WAVES waves (4 as
// launched) of 32 queries of one (b, h).  K and V tiles of 64 keys are
// double-buffered in LDS, moved there by LDS-DMA one tile ahead.  Scores are
// computed transposed, S^T = K * Q^T, with v_mfma_f32_32x32x16_bf16: Q^T is
// the B operand and stays in registers for the whole key loop, and each
// lane's accumulator column is one query, so the softmax max/sum over keys is
// an in-lane reduction plus one exchange with lane ^ 32.  The probabilities
// are rounded to bf16 and fed, in exactly the registers the score MFMA wrote
// them to, as the B operand of O^T += V^T * P^T; V stays row-major in LDS and
// the V^T operand is read with ds_read_b64_tr_b16 (two 8-byte transposing
// reads per MFMA).  A wave's VALU work does not overlap its own MFMAs, only
// another wave's, so the softmax is pared down: the tile max is taken on raw
// scores, scale * log2 e and the max subtraction are one FMA ahead of
// v_exp_f32, the running output is rescaled only when the max grows by more
// than 2^8 (a wave-uniform branch, normally taken on the first tile only),
// and probabilities are rounded to bf16 two per v_cvt_pk_bf16_f32.  fp32
// throughout; the output is normalised once at the end.  Causal tiles beyond
// a wave's last query are skipped per wave and the query-block order is
// reversed so the heaviest blocks start first.
// The 1-D grid is remapped so that each XCD runs the query blocks of a few
// (b, h) pairs at a time: they stream the same K/V tiles, which then come
// from that XCD's L2 rather than once per workgroup from HBM.
//
// fa_fwd_rows (fp32 at any power-of-two head_dim <= 256, and bf16 at the
// head sizes the MFMA kernel does not take: 16, 32, 256).  The reference's
// per-query-row structure — grid (N_q, BH), one wave per query row — with
// the key loop vectorised across lanes: each lane scores one key of a
// 64-key chunk, and the chunk is folded into the running (m, l, acc) state.
// bf16 operands are widened to fp32 on load; all arithmetic is fp32.
#include "mfma.hpp"

namespace teeny {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
// Largest growth (log2 units) of a tile max over the reference point before
// the running output is rescaled: probabilities stay <= 2^8.
constexpr float kRescale = 8.0f;
#ifndef ATTN_LA
#define ATTN_LA 3
#endif

template <int D, bool CAUSAL, int WAVES>
__global__ __launch_bounds__(64 * WAVES, 8 / WAVES) void fa_fwd_bf16(const bf16 *__restrict__ Q,
                                                      const bf16 *__restrict__ K,
                                                      const bf16 *__restrict__ V,
                                                      bf16 *__restrict__ O, float *__restrict__ L,
                                                      int nq, int nk, float scale_log2, int nqb,
                                                      int kv_group) {
  constexpr int NT = 64 * WAVES;   // threads per workgroup
  constexpr int BM = 32 * WAVES;   // queries per workgroup (32 per wave)
  constexpr int BN = 64;           // keys per tile
  constexpr int CPR = D / 8;       // 16-byte chunks per K/V row
  constexpr int RPB = 128 / D;     // rows per 256-byte LDS bank window
  constexpr int RPI = NT / CPR;    // rows covered by one load round of the workgroup
  constexpr int NLD = BN * CPR / NT;  // load rounds per tile
  constexpr int TILE = BN * D;     // elements of one K or V tile
  constexpr int NS = D / 16;       // k-steps of the score MFMA
  constexpr int ND = D / 32;       // d-blocks of the output
  static_assert(NLD >= 1 && BN * CPR % NT == 0, "tile must be a whole number of load rounds");
  // K tiles (t & 1) then V tiles (t & 1), dense rows with XOR-swizzled
  // 16-byte chunks: chunk j of row r sits at position j ^ fk(r) (K) or
  // j ^ fv(r) (V).  fk spreads the 16 rows that one ds_read_b128 quarter-wave
  // touches over all 64 banks; fv does the same for the 4 rows x 64 bytes
  // that a half-wave of ds_read_b64_tr_b16 touches.
  // Four separate arrays, and every use picks one by a compile-time parity,
  // so the compiler can tell that a stage's LDS reads never alias the DMA
  // it has just started into the other buffer (otherwise it waits for that
  // DMA before the first read).
  __shared__ __attribute__((aligned(16))) bf16 kbuf0[TILE], kbuf1[TILE], vbuf0[TILE], vbuf1[TILE];
  auto kbuf = [&](auto par) -> bf16 * { if constexpr (decltype(par)::value) return kbuf1; else return kbuf0; };
  auto vbuf = [&](auto par) -> bf16 * { if constexpr (decltype(par)::value) return vbuf1; else return vbuf0; };
  auto fk = [](int row) { return (row / RPB) & (CPR - 1); };
  auto fv = [](int row) { return (4 * (row / RPB)) & (CPR - 1) & ~3; };

  // All query blocks of one (b, h) are consecutive logical ids on one XCD,
  // so they run together and read K/V once from HBM into that XCD's L2.
  // Causal: a query block's work grows with its index, so workgroup p of a
  // head runs blocks nqb-1-p and then p, and every workgroup does the same
  // nqb + 1 key tiles (balanced by construction, whatever the dispatch order).
  const int tile_id = xcd_remap(blockIdx.x, gridDim.x);
  const int per_bh = CAUSAL ? (nqb + 1) / 2 : nqb;
  const int bh = tile_id / per_bh;
  const int slot = tile_id % per_bh;
  const int npass = CAUSAL && slot < nqb - 1 - slot ? 2 : 1;
  for (int pass = 0; pass < npass; ++pass) {
    const int qb = pass == 0 ? nqb - 1 - slot : slot;
    // opaque per pass: nothing derived from the thread id is hoisted out of
    // the pass loop into registers that would stay live across it
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    const int w = tid >> 6, lane = tid & 63, g = lane >> 5, c = lane & 31;
    const int q0 = qb * BM + w * 32;
    const int qi = q0 + c;

    const bf16 *Qb = Q + static_cast<int64_t>(bh) * nq * D;
    // grouped-query attention: kv_group consecutive query heads share one K/V head
    const bf16 *Kb = K + static_cast<int64_t>(bh / kv_group) * nk * D;
    const bf16 *Vb = V + static_cast<int64_t>(bh / kv_group) * nk * D;

    // A negative softmax scale is applied by negating Q (exact in bf16), so the
    // score multiplier sc is positive and the running max is a max.  It is at
    // least FLT_MIN so that a masked -inf score maps to p = 0 even for a zero
    // scale (where every finite score then gives p = 1 exactly, as it should).
    const float sc = fmaxf(fabsf(scale_log2), 1.17549435e-38f);
    const uint32_t qsign = scale_log2 < 0.0f ? 0x80008000u : 0u;
    bf16x8 qf[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      u32x4 raw = u32x4{0u, 0u, 0u, 0u};
      if (qi < nq) raw = *reinterpret_cast<const u32x4 *>(Qb + static_cast<int64_t>(qi) * D + 16 * s + 8 * g);
      raw ^= qsign;
      __builtin_memcpy(&qf[s], &raw, 16);
    }

    f32x16 acc[ND];
#pragma unroll
    for (int d = 0; d < ND; ++d) acc[d] = zero16();
    // m_run: reference point of the exponentials (log2 domain, already scaled).
    // It is raised only when a tile's max exceeds it by more than kRescale, so
    // p = 2^(sc*s - m_run) <= 2^kRescale and O is rescaled on few tiles.
    float m_run = -INFINITY, l_run = 0.0f;
    const int kv_end = CAUSAL ? min(nk, qb * BM + BM) : nk;
    const int n_tiles = (kv_end + BN - 1) / BN;
    const int wave_end = CAUSAL ? min(kv_end, q0 + 32) : kv_end;

    // ── global -> LDS: one 16-byte slot per thread per round, straight into
    // LDS by buffer loads with the lds flag (lane j of a wave lands at
    // base + 16 j).  Slot t + NT i of a tile is row t / CPR + RPI i, position
    // t % CPR; the source chunk is that position XOR the row's swizzle.  The
    // buffer extent is the head's nk rows, so rows past nk read as zeros and
    // P = 0 never meets stale data in the P*V product.  The DMA is issued from
    // inline assembly: the compiler's own tracking of an LDS DMA in flight
    // turns every LDS-read wait of the stage into lgkmcnt(0).
    const int ld_row = tid / CPR;
    const int k_off = 2 * (ld_row * D + ((tid % CPR) ^ fk(ld_row)) * 8);
    const int v_off = 2 * (ld_row * D + ((tid % CPR) ^ fv(ld_row)) * 8);
    const __amdgpu_buffer_rsrc_t k_rsrc = buffer_rsrc(Kb, nk * D * 2);
    const __amdgpu_buffer_rsrc_t v_rsrc = buffer_rsrc(Vb, nk * D * 2);
    auto load_tile = [&](__amdgpu_buffer_rsrc_t r, bf16 *dst, int kbase, int off) __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < NLD; ++i)
        buffer_lds_dma16(r, off + 2 * (kbase + RPI * i) * D,
                         __builtin_amdgcn_readfirstlane(lds_address(dst + (NT * i + 64 * w) * 8)));
    };

    // ── LDS -> operands
    // K (A operand of S^T = K Q^T): lane (g, c) reads row kb*32 + c, chunk
    // 2 st + g, i.e. element offset koff(st) = kofs ^ (st << 4).
    // V^T (A operand of O^T += V^T P^T) through ds_read_b64_tr_b16: in each
    // 16-lane group, lane i receives element i & 3 of the 8-byte pieces
    // addressed by lanes (i >> 2) + 4 j, j = 0..3.  Lane m of group h points
    // at key 8 r + 4 g + (m >> 2) (plus kb*32 + 16 tt) and d = 32 dblk +
    // 16 (h & 1) + 4 (m & 3), so lane l receives d = 32 dblk + l % 32 for the
    // four keys that its P registers hold; offset voff(dblk) = vofs ^ (dblk << 5).
    // In both, the step-dependent part is an XOR on offset bits that the row
    // part does not touch, so each fragment address is one v_xor_b32 from a
    // single per-lane base (cheaper than holding NS + ND offsets in registers).
    static_assert(D == 64 || D == 128, "offset XOR layout assumes D of 64 or 128");
    const int hh = lane >> 4, m16 = lane & 15;
    const int v_row = 4 * g + (m16 >> 2);
    int kofs = c * D + ((g ^ fk(c)) << 3);
    int vofs = v_row * D + ((fv(v_row) | (2 * (hh & 1) + ((m16 & 3) >> 1))) << 3) + (m16 & 1) * 4;

    // S^T for key tile kt (K from LDS as the A operand, Q^T from registers).
    auto score = [&](auto par, f32x16 (&s)[2]) __attribute__((always_inline)) {
      const bf16 *ks = kbuf(par);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        s[kb] = zero16();
#pragma unroll
        for (int st = 0; st < NS; ++st) {
          const bf16x8 a = *reinterpret_cast<const bf16x8 *>(ks + kb * 32 * D + (kofs ^ (st << 4)));
          s[kb] = mfma32x32x16(a, qf[st], s[kb]);
        }
      }
    };

    // Software pipeline, one barrier per key tile.  Iteration kt starts the
    // loads of K for tile kt+2 and V for tile kt+1 (each into the buffer whose
    // last reader finished before the previous barrier), computes the scores
    // of tile kt+1 on the matrix cores while the softmax of tile kt runs on the
    // VALU, accumulates P*V of tile kt, and waits for its own loads before the
    // barrier that publishes them.
    const std::false_type even{};
    const std::true_type odd{};
    load_tile(k_rsrc, kbuf(even), 0, k_off);
    if (n_tiles > 1) load_tile(k_rsrc, kbuf(odd), BN, k_off);
    load_tile(v_rsrc, vbuf(even), 0, v_off);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    // Masks tile kt of a wave's scores (keys past nk; causal: keys past the
    // query) and returns the raw max over the tile for each query lane.
    auto mask_scores = [&](int kt, f32x16 (&sc_t)[2]) __attribute__((always_inline)) {
      const int kbase = kt * BN;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int key = kbase + kb * 32 + mfma32_row(v, g);
          if (key >= nk || (CAUSAL && key > qi)) sc_t[kb][v] = -INFINITY;
        }
    };
    auto tile_max = [&](const f32x16 (&sc_t)[2]) __attribute__((always_inline)) {
      // Three-input tree (v_maximum3_f32: 17 instructions for 32 values).
      // IEEE maximum rather than fmaxf: fmaxf's NaN-dropping form makes the
      // compiler canonicalize every MFMA result first (one extra VALU op per
      // score); a NaN score gives a NaN row either way, through p.
      auto mx2 = [](float a, float b) { return __builtin_elementwise_maximum(a, b); };
      auto mx3 = [&](float a, float b, float c) { return mx2(mx2(a, b), c); };
      float x[32];
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        x[v] = sc_t[0][v];
        x[16 + v] = sc_t[1][v];
      }
      float u[11];
#pragma unroll
      for (int i = 0; i < 10; ++i) u[i] = mx3(x[3 * i], x[3 * i + 1], x[3 * i + 2]);
      u[10] = mx2(x[30], x[31]);
      const float w0 = mx3(u[0], u[1], u[2]), w1 = mx3(u[3], u[4], u[5]), w2 = mx3(u[6], u[7], u[8]);
      const float mx = mx3(mx3(w0, w1, w2), u[9], u[10]);
      // the keys of a query are split over lanes l and l ^ 32
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
      return mx2(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
    };
    auto needs_mask = [&](int kt) {
      return (kt * BN + BN > nk) || (CAUSAL && kt * BN + BN - 1 > q0);
    };

    // One pipeline stage.  On entry s_cur holds the masked scores of tile kt
    // and mx_cur their max; the stage leaves the same for tile kt+1 in s_nx and
    // mx_cur.  The scores of tile kt+1 are computed unconditionally (past the
    // last tile they read a stale, in-bounds K buffer and are never used).  The
    // loop below is unrolled by two so that the two score buffers swap roles
    // without register copies, and each stage body is one straight-line block
    // in which the VALU work (this tile's exponentials) can issue in the
    // shadow of the 32 MFMAs; the next tile's max closes the stage.
    float mx_cur = -INFINITY;
    // par is the parity of kt (compile time: the loop is unrolled by two).
    auto stage = [&](auto par, int kt, f32x16 (&s_cur)[2], f32x16 (&s_nx)[2]) __attribute__((always_inline)) {
      constexpr bool P = decltype(par)::value;
      const std::integral_constant<bool, !P> npar{};
      if (kt + 2 < n_tiles) load_tile(k_rsrc, kbuf(par), (kt + 2) * BN, k_off);
      if (kt + 1 < n_tiles) load_tile(v_rsrc, vbuf(npar), (kt + 1) * BN, v_off);

      if (kt * BN < wave_end) {  // causal: later tiles are beyond this wave's last query
        const float mx_s = mx_cur * sc;  // sc > 0: -inf stays -inf
        if (__any(mx_s > m_run + kRescale)) {
          const float m_new = fmaxf(m_run, mx_s);
          const float alpha = __builtin_amdgcn_exp2f(m_run - (m_new == -INFINITY ? 0.0f : m_new));
          l_run *= alpha;
#pragma unroll
          for (int d = 0; d < ND; ++d)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[d][v] *= alpha;
          m_run = m_new;
        }
        const float neg_m = m_run == -INFINITY ? 0.0f : -m_run;

        auto body = [&]() __attribute__((always_inline)) {
          // Hand-pipelined block of 2 NS score MFMAs (next tile) followed by
          // 4 ND P*V MFMAs (this tile).  Each bundle is one MFMA, the LDS
          // read(s) for the MFMA kLA bundles later (into a rotating window of
          // kW fragments) and a slice of the softmax VALU work; a
          // sched_barrier after each bundle keeps this order, so the reads
          // stay kLA MFMAs ahead and the window registers are never reused
          // while a read into them is in flight.
          constexpr int kLA = ATTN_LA, kW = kLA + 1;
          constexpr int nS = 2 * NS, nPV = 4 * ND;
          constexpr int PPB = 16 / nS;  // softmax value pairs per score bundle
          const bf16 *ks = kbuf(npar);
          const bf16 *vs = vbuf(par);
          // opaque per stage: the fragment addresses are re-derived here (one
          // XOR each) rather than hoisted out of the loop into registers
          int kofs_s = kofs, vofs_s = vofs;
          asm volatile("" : "+v"(kofs_s), "+v"(vofs_s));
          bf16x8 kw[kW];
          bf16x4 vw[kW][2];
          // score MFMA i: key block kb = i / NS, k-step st = i % NS
          auto kread = [&](int i) __attribute__((always_inline)) {
            kw[i % kW] = *reinterpret_cast<const bf16x8 *>(ks + (i / NS) * 32 * D + (kofs_s ^ ((i % NS) << 4)));
          };
          // P*V MFMA j: d-block d = j % ND, then tt, then kb
          auto vread = [&](int j) __attribute__((always_inline)) {
            const int d = j % ND, tt = (j / ND) & 1, kb = j / (2 * ND);
            const bf16 *vp = vs + (kb * 32 + 16 * tt) * D + (vofs_s ^ (d << 5));
            vw[j % kW][0] = ds_read_tr16(vp);
            vw[j % kW][1] = ds_read_tr16(vp + 8 * D);
          };
          // p = 2^(sc * s - m_run) (0 for masked keys), rounded to bf16
          // pairwise into exactly the registers of the B operand of the P*V
          // product; the row sum stays in fp32 so that L = m + log(l) keeps
          // fp32 accuracy.
          u32x4 pw[2][2];
          // four partial sums, each started by its first pair (no + 0.0f,
          // which the compiler must keep for a -0.0 operand)
          float ps[4];
          auto softmax_pair = [&](int q) __attribute__((always_inline)) {
            const int kb = q >> 3, v = 2 * (q & 7);
            const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s_cur[kb][v], sc, neg_m));
            const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s_cur[kb][v + 1], sc, neg_m));
            if (q < 4) ps[q & 3] = p0 + p1;
            else ps[q & 3] += p0 + p1;
            // the sum is taken here, not after the last MFMA: otherwise all
            // 32 fp32 p of the tile stay live across the stage
            asm volatile("" : "+v"(ps[q & 3]));
            const bf16x2 pair = cvt_pk_bf16(p0, p1);
            uint32_t word;
            __builtin_memcpy(&word, &pair, 4);
            pw[kb][v >> 3][(v & 7) >> 1] = word;
          };

#pragma unroll
          for (int i = 0; i < kLA; ++i) kread(i);
          // Wave priority 1 over the score bundles, 0 over P*V and the tail:
          // of the two waves on a SIMD, the one issuing score MFMAs with
          // exponentials in between is issued first, and the P*V MFMAs of
          // the other fill the matrix core around it (5% fewer cycles per
          // tile measured).
          __builtin_amdgcn_s_setprio(1);
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int i = 0; i < nS; ++i) {
            const int ahead = i + kLA;
            if (ahead < nS) kread(ahead);
            else vread(ahead - nS);
            const int kb = i / NS, st = i % NS;
            s_nx[kb] = mfma32x32x16(kw[i % kW], qf[st], st == 0 ? zero16() : s_nx[kb]);
#pragma unroll
            for (int q = 0; q < PPB; ++q) softmax_pair(i * PPB + q);
            __builtin_amdgcn_sched_barrier(0);
          }
          l_run += (ps[0] + ps[1]) + (ps[2] + ps[3]);
          __builtin_amdgcn_s_setprio(0);
#pragma unroll
          for (int j = 0; j < nPV; ++j) {
            if (j + kLA < nPV) vread(j + kLA);
            const int d = j % ND, tt = (j / ND) & 1, kb = j / (2 * ND);
            bf16x8 pb;
            __builtin_memcpy(&pb, &pw[kb][tt], 16);
            acc[d] = mfma32x32x16(cat8(vw[j % kW][0], vw[j % kW][1]), pb, acc[d]);
            __builtin_amdgcn_sched_barrier(0);
          }

          // rare (last tile, causal diagonal): a wave-uniform branch after
          // every MFMA of the stage has issued
          if (needs_mask(kt + 1)) {
            asm volatile("" ::: "memory");
            mask_scores(kt + 1, s_nx);
          }
          mx_cur = tile_max(s_nx);
        };
        body();
      }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
    };

    f32x16 sa[2], sb[2];
    score(even, sa);
    if (needs_mask(0)) mask_scores(0, sa);
    mx_cur = tile_max(sa);
    __syncthreads();  // K buffer 0 is reloaded (tile 2) at the start of stage 0
    for (int kt = 0; kt < n_tiles; kt += 2) {
      stage(even, kt, sa, sb);
      if (kt + 1 >= n_tiles) break;
      stage(odd, kt + 1, sb, sa);
    }

    const auto lsw = __builtin_amdgcn_permlane32_swap(__float_as_uint(l_run), __float_as_uint(l_run), false, false);
    const float l_tot = __uint_as_float(lsw[0]) + __uint_as_float(lsw[1]);
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
  }  // pass
}

// Per-row path: grid (nq, BH), one wave per query row (flash_attn2.rs:48-51).
template <typename T, int D>
__global__ __launch_bounds__(64) void fa_fwd_rows(const T *__restrict__ Q, const T *__restrict__ K,
                                                  const T *__restrict__ V, T *__restrict__ O,
                                                  float *__restrict__ L, int nq, int nk, float scale, int causal,
                                                  int kv_group) {
  constexpr int DPL = (D + 63) / 64;  // output elements per lane
  __shared__ float qs[D];
  __shared__ float ps[64];
  const int qi = blockIdx.x;
  const int64_t bh = blockIdx.y;
  const int lane = threadIdx.x;
  const T *qrow = Q + (bh * nq + qi) * D;
  const T *Kb = K + (bh / kv_group) * nk * D;
  const T *Vb = V + (bh / kv_group) * nk * D;
  for (int d = lane; d < D; d += 64) qs[d] = to_f32(qrow[d]);
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
      const T *krow = Kb + static_cast<int64_t>(key) * D;
      float dot = 0.0f;
#pragma unroll 8
      for (int d = 0; d < D; ++d) dot += qs[d] * to_f32(krow[d]);
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
        for (int j = 0; j < cnt; ++j) a += ps[j] * to_f32(Vb[static_cast<int64_t>(k0 + j) * D + d]);
        acc[i] = a;
      }
    }
    m_i = m_new;
    __syncthreads();
  }
  T *orow = O + (bh * nq + qi) * D;
#pragma unroll
  for (int i = 0; i < DPL; ++i) {
    const int d = lane + 64 * i;
    if (d < D) orow[d] = from_f32<T>(acc[i] / l_i);
  }
  if (L != nullptr && lane == 0) L[bh * nq + qi] = m_i + logf(l_i);
}

template <typename T, int D>
static void launch_rows(const void *q, const void *k, const void *v, void *o, float *l, int nq,
                        int nk, float scale, int BH, int causal, int kv_group, hipStream_t s) {
  hipLaunchKernelGGL((fa_fwd_rows<T, D>), dim3(nq, BH), dim3(64), 0, s, static_cast<const T *>(q),
                     static_cast<const T *>(k), static_cast<const T *>(v), static_cast<T *>(o), l, nq, nk,
                     scale, causal, kv_group);
}

template <int D>
static void launch_bf16(const void *q, const void *k, const void *v, void *o, float *l, int nq,
                        int nk, float scale, int BH, int causal, int kv_group, hipStream_t s) {
  constexpr int WAVES = 4;
  const int nqb = (nq + 32 * WAVES - 1) / (32 * WAVES);
  const float scale_log2 = scale * kLog2e;
  const dim3 grid(BH * (causal ? (nqb + 1) / 2 : nqb));
  if (causal) {
    hipLaunchKernelGGL((fa_fwd_bf16<D, true, WAVES>), grid, dim3(64 * WAVES), 0, s,
                       static_cast<const bf16 *>(q), static_cast<const bf16 *>(k),
                       static_cast<const bf16 *>(v), static_cast<bf16 *>(o), l, nq, nk, scale_log2,
                       nqb, kv_group);
  } else {
    hipLaunchKernelGGL((fa_fwd_bf16<D, false, WAVES>), grid, dim3(64 * WAVES), 0, s,
                       static_cast<const bf16 *>(q), static_cast<const bf16 *>(k),
                       static_cast<const bf16 *>(v), static_cast<bf16 *>(o), l, nq, nk, scale_log2,
                       nqb, kv_group);
  }
}

// Shared by both entry points: q [batch * q_heads, nq, D], k/v
// [batch * kv_heads, nk, D]; query head h of a batch reads K/V head
// h / (q_heads / kv_heads).
static teeny_status attention_entry(const void *q, const void *k, const void *v, void *o, float *l,
                                    int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t n_ctx_q,
                                    int64_t n_ctx_k, int64_t head_dim, float softmax_scale, int32_t causal,
                                    teeny_dtype dtype, teeny_stream stream, const char *name) {
  const std::string nm(name);
  TEENY_REQUIRE(n_ctx_q >= 0 && n_ctx_k >= 0 && batch >= 0 && q_heads >= 0 && kv_heads >= 0,
                TEENY_ERR_SHAPE_MISMATCH, nm + ": negative size");
  TEENY_REQUIRE(kv_heads > 0 ? q_heads % kv_heads == 0 : q_heads == 0, TEENY_ERR_SHAPE_MISMATCH,
                nm + ": q_heads must be a multiple of kv_heads");
  const int64_t BH = batch * q_heads;
  if (n_ctx_q == 0 || BH == 0) return TEENY_OK;
  TEENY_REQUIRE(n_ctx_k > 0, TEENY_ERR_SHAPE_MISMATCH, nm + ": n_ctx_k must be positive (softmax over no keys)");
  TEENY_REQUIRE(n_ctx_q <= 0x7fffffff && n_ctx_k <= 0x7fffffff && BH <= 65535 &&
                    BH * ((n_ctx_q + 127) / 128) <= 0x7fffffff,
                TEENY_ERR_SHAPE_MISMATCH, nm + ": size out of range");
  TEENY_REQUIRE(q != nullptr && k != nullptr && v != nullptr && o != nullptr, TEENY_ERR_NULL_POINTER,
                nm + ": q/k/v/o");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int nq = static_cast<int>(n_ctx_q), nk = static_cast<int>(n_ctx_k);
  const int bh = static_cast<int>(BH), group = static_cast<int>(q_heads / kv_heads);
  if (dtype == TEENY_F32) {
    switch (head_dim) {
      case 16: launch_rows<float, 16>(q, k, v, o, l, nq, nk, softmax_scale, bh, causal, group, s); break;
      case 32: launch_rows<float, 32>(q, k, v, o, l, nq, nk, softmax_scale, bh, causal, group, s); break;
      case 64: launch_rows<float, 64>(q, k, v, o, l, nq, nk, softmax_scale, bh, causal, group, s); break;
      case 128: launch_rows<float, 128>(q, k, v, o, l, nq, nk, softmax_scale, bh, causal, group, s); break;
      case 256: launch_rows<float, 256>(q, k, v, o, l, nq, nk, softmax_scale, bh, causal, group, s); break;
      default: return fail(TEENY_ERR_UNSUPPORTED, nm + ": f32 head_dim must be 16, 32, 64, 128 or 256");
    }
    return after_launch(name, s);
  }
  if (dtype == TEENY_BF16) {
    switch (head_dim) {  // head sizes off the matrix-core kernel: the per-row kernel
      case 16: launch_rows<bf16, 16>(q, k, v, o, l, nq, nk, softmax_scale, bh, causal, group, s); break;
      case 32: launch_rows<bf16, 32>(q, k, v, o, l, nq, nk, softmax_scale, bh, causal, group, s); break;
      case 256: launch_rows<bf16, 256>(q, k, v, o, l, nq, nk, softmax_scale, bh, causal, group, s); break;
      case 64:
      case 128: break;
      default: return fail(TEENY_ERR_UNSUPPORTED, nm + ": bf16 head_dim must be 16, 32, 64, 128 or 256");
    }
    if (head_dim != 64 && head_dim != 128) return after_launch(name, s);
    TEENY_REQUIRE(aligned(q, 16) && aligned(k, 16) && aligned(v, 16) && aligned(o, 16),
                  TEENY_ERR_MISALIGNED, nm + ": bf16 q/k/v/o must be 16-byte aligned");
    // K and V of one (batch, head) are read through 32-bit buffer offsets
    TEENY_REQUIRE(n_ctx_k * head_dim * 2 <= 0x7fffffff, TEENY_ERR_SHAPE_MISMATCH,
                  nm + ": bf16 K/V of one head must be below 2 GiB");
    if (head_dim == 64) launch_bf16<64>(q, k, v, o, l, nq, nk, softmax_scale, bh, causal, group, s);
    else launch_bf16<128>(q, k, v, o, l, nq, nk, softmax_scale, bh, causal, group, s);
    return after_launch(name, s);
  }
  return fail(TEENY_ERR_UNSUPPORTED_DTYPE, nm + ": dtype must be F32 or BF16");
}

}  // namespace teeny

using namespace teeny;

extern "C" teeny_status teeny_flash_attention2_forward(const void *q, const void *k, const void *v,
                                                       void *o, float *l, int64_t n_ctx_q,
                                                       int64_t n_ctx_k, float softmax_scale,
                                                       int64_t BH, int64_t head_dim,
                                                       int32_t causal, teeny_dtype dtype,
                                                       teeny_stream stream) {
  return attention_entry(q, k, v, o, l, BH, 1, 1, n_ctx_q, n_ctx_k, head_dim, softmax_scale, causal, dtype,
                         stream, "flash_attention2_forward");
}

extern "C" teeny_status teeny_attention_forward(const void *q, const void *k, const void *v, void *o,
                                                float *l, int64_t batch, int64_t q_heads, int64_t kv_heads,
                                                int64_t n_ctx_q, int64_t n_ctx_k, int64_t head_dim,
                                                float softmax_scale, int32_t causal, teeny_dtype dtype,
                                                teeny_stream stream) {
  return attention_entry(q, k, v, o, l, batch, q_heads, kv_heads, n_ctx_q, n_ctx_k, head_dim, softmax_scale,
                         causal, dtype, stream, "attention_forward");
}
