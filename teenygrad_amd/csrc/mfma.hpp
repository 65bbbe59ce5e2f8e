// gfx950 MFMA fragment conventions used by the attention, GEMM and conv kernels.
//
// v_mfma_f32_32x32x16_bf16 (one wave64):  D[32x32] += A[32x16] * B[16x32]
//   A: lane l holds A[l % 32][8 * (l / 32) + j], j = 0..7   (bf16x8)
//   B: lane l holds B[8 * (l / 32) + j][l % 32], j = 0..7   (bf16x8)
//   D: lane l holds D[8 * (v / 4) + 4 * (l / 32) + (v % 4)][l % 32], v = 0..15
// Only the D layout matters for correctness of a kernel that builds A and B
// with the same k assignment: the k order inside one instruction is a
// permutation shared by A and B and cancels in the sum.
#pragma once

#include "common.hpp"

namespace teeny {

// Raw buffer resource over [base, base + bytes): a load at an offset past
// the extent returns zeros.  kOffNone is such an offset for any extent below
// 2^31.  Word 3 is the gfx9 raw-buffer format (32-bit data, no swizzle).
constexpr uint32_t kBufWord3 = 0x00020000u;
constexpr int kOffNone = static_cast<int>(0x80000000u);
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void *base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, bytes, kBufWord3);
}
__device__ __forceinline__ u32x4 buffer_load16(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

__device__ __forceinline__ uint32_t lds_address(const void *p) {
  typedef __attribute__((address_space(3))) const char lds_char;
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_char *)(p)));
}

// One 16-byte LDS-DMA per lane from a buffer resource: lane j writes
// lds + 16 j, reading [voff, voff + 16) (zeros past the extent).  M0 carries
// the wave's LDS base and is restored afterwards.  Issued from inline
// assembly, so the compiler neither tracks it (the caller waits on vmcnt
// itself) nor lets it degrade its own LDS-read waits to lgkmcnt(0).
// s_waitcnt immediate that waits until at most n vector memory operations
// are outstanding (gfx9 encoding: vmcnt in bits 3:0 and 15:14, expcnt and
// lgkmcnt left at their maxima, i.e. not waited for).
constexpr int vm_wait(int n) { return 0xF70 | (n & 15) | ((n >> 4) << 14); }

__device__ __forceinline__ void buffer_lds_dma16(__amdgpu_buffer_rsrc_t r, int voff, uint32_t lds) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %3\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %1, %2, 0 offen lds\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(voff), "s"(r), "s"(lds)
      : "memory");
}

__device__ __forceinline__ f32x16 mfma32x32x16(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Row of the D fragment held in register v by lane group g = lane / 32.
__device__ __forceinline__ constexpr int mfma32_row(int v, int g) {
  return 8 * (v >> 2) + 4 * g + (v & 3);
}

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.0f;
  return z;
}

// Concatenates two 4-element bf16 vectors (two 8-byte LDS reads) into one operand.
__device__ __forceinline__ bf16x8 cat8(bf16x4 lo, bf16x4 hi) {
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

// Rounds two floats to bf16 (nearest-even) with one v_cvt_pk_bf16_f32.
__device__ __forceinline__ bf16x2 cvt_pk_bf16(float a, float b) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  return __builtin_convertvector((f32x2){a, b}, bf16x2);
}

// ds_read_b64_tr_b16: within each group of 16 lanes, lane i receives
// element i & 3 of the 8-byte pieces addressed by lanes (i >> 2) + 4 j,
// j = 0..3 (a 4x4 transpose of 16-bit elements per quarter of the group).
__device__ __forceinline__ bf16x4 ds_read_tr16(const bf16 *p) {
  typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4 *)(p));
}

// Chunk swizzle of LDS tile rows (64 banks of 4 bytes: one 256-byte window).
// A ds_read_b128 is served 16 lanes at a time and a ds_read_b64(_tr_b16) 32
// lanes at a time, so the swizzle must give
//   * row reads (frag_row): 16 consecutive rows, one logical chunk -> 16
//     distinct 16-byte positions of the window;
//   * transposing reads (frag_tr): 4 consecutive rows x 4 adjacent chunks
//     (one 64-byte column block) -> 16 distinct positions.
// D = 128 (one row per window): position = chunk ^ (4 (row % 4) + (row / 4) % 4),
// whose high two bits differ across 4 consecutive rows.  D = 64 (two rows per
// window, row parity picks the half): the same with k = (row / 2) % 8,
// 4 (k % 2) + k / 2, so rows r and r + 2 use opposite 64-byte column halves.
template <int D>
__device__ __forceinline__ int bswz(int row) {
  if constexpr (D == 128) {
    const int h = row & 15;
    return ((h & 3) << 2) | ((h >> 2) & 3);
  } else {
    const int k = (row >> 1) & 7;
    return ((k & 1) << 2) | ((k >> 1) & 3);
  }
}

// Transposed A operand: lane (g, r) holds column d = 32 db + r of tile rows
// rb + {4g .. 4g+3, 8+4g .. 8+4g+3} (rb a multiple of 16) — the k order of a
// 32x32 result's registers 8t .. 8t+7 packed as a B operand (pack_b).  Two
// ds_read_b64_tr_b16: lane m of each 16-lane group addresses row
// rb + 4g + m/4 (+ 8), columns 32 db + 16 (group & 1) + 4 (m & 3) .. + 3.
template <int D>
__device__ __forceinline__ bf16x8 frag_tr(const bf16 *tile, int rb, int db, int lane) {
  constexpr int HI = 2;  // bswz(row + 8) = bswz(row) ^ 2 for row % 16 < 8 (both D)
  const int g = lane >> 5, hh = lane >> 4, m = lane & 15;
  const int rr = 4 * g + (m >> 2);
  const int cc = 4 * db + 2 * (hh & 1) + ((m & 3) >> 1);
  const int sw = bswz<D>(rr);
  const bf16 *p0 = tile + (rb + rr) * D + ((cc ^ sw) << 3) + 4 * (m & 1);
  const bf16 *p1 = tile + (rb + 8 + rr) * D + ((cc ^ sw ^ HI) << 3) + 4 * (m & 1);
  return cat8(ds_read_tr16(p0), ds_read_tr16(p1));
}

// Packs two bf16 bit patterns (low halves of a and b) into one 32-bit word.
__device__ __forceinline__ uint32_t pack_lo(uint32_t a, uint32_t b) {
  return (a & 0xffffu) | (b << 16);
}
__device__ __forceinline__ uint32_t pack_hi(uint32_t a, uint32_t b) {
  return (a >> 16) | (b & 0xffff0000u);
}

}  // namespace teeny
