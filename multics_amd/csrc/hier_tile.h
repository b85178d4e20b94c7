// Shared machinery of the attention kernels: 64-row LDS tiles of bf16 rows
// (keys for the forward; keys or queries for the backward) copied straight
// from HBM / L2 into LDS with global_load_lds_dwordx4, and the MFMA operand
// reads out of them.
//
// Layout of a tile: rows of 2*D bytes with no padding.  Row j of a 16-row
// group sits at position NR*(j % NI) + j / NI of the group (NI = D/32 copy
// instructions per wave, NR = 64 lanes / (D/8) chunks = rows per copy
// instruction), so each lane copies NI consecutive rows of one row slot.  The
// 16-byte chunks of a row are XOR-swizzled per row, with one of three
// swizzles chosen by how the tile is read:
//   kRowRead   16 consecutive rows at one chunk column (ds_read_b128, the row
//              operand of an MFMA);
//   kTrRead    4 rows x 4 chunks per 32 lanes (ds_read_b64_tr_b16, the
//              transposed operand);
//   kBothRead  both patterns.
// Each is free of bank conflicts for its pattern(s).  All three are linear
// over GF(2) in the row bits, so the chunk of copy e of a lane is the lane's
// base chunk XOR swz(e).
#pragma once

#include "hier_common.h"

namespace hier {
namespace tile {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

constexpr int kSlab = 64;   // rows per LDS tile

template <int D>
struct Geo {
  static constexpr int ROWB = 2 * D;                // bytes per row
  static constexpr int CPR = D / 8;                 // 16-byte chunks per row
  static constexpr int NI = D / 32;                 // copy instructions per wave per tile
  static constexpr int NR = 64 / CPR;               // rows per copy instruction
  static constexpr int TILEB = kSlab * ROWB;
  static constexpr int MBYTES = kSlab * 4;          // one dword per row
  static constexpr int NC = D / 16;                 // 16-wide d-chunks (MFMA K steps over d)
  static constexpr int NDB = D / 32;                // 32-wide d-blocks (MFMA rows over d)
  static_assert(NI * NR == 16, "a wave copies 16 rows per tile");
};

enum Swizzle { kRowRead = 0, kTrRead = 1, kBothRead = 2 };

// Position of row `row` inside its tile.
template <int D>
__device__ __forceinline__ constexpr int prow(int row) {
  return (row & ~15) + Geo<D>::NR * ((row & 15) % Geo<D>::NI) + (row & 15) / Geo<D>::NI;
}

// XOR mask on the 16-byte chunk index of row `row`.
template <int D, int S>
__device__ __forceinline__ constexpr int swz(int row) {
  if (S == kRowRead) return D == 128 ? (row & 15) : ((row & 1) | ((row >> 1) & 6));
  if (S == kTrRead) return D == 128 ? 4 * (row & 3) : 4 * (row & 1);
  return D == 128 ? (((row & 3) << 2) | ((row >> 2) & 3)) : (((row & 1) << 2) | ((row >> 2) & 3));
}

__device__ __forceinline__ float pair_max(float v) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float v) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ uint32_t wave_or(uint32_t v) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) v |= __shfl_xor(v, d, 64);
  return v;
}
__device__ __forceinline__ uint16_t f2bf(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);  // round to nearest even
}

// ---- tile copies (global -> LDS) -------------------------------------------

// Per-lane constants of the tile copies: the lane copies chunk pc of row slot
// r for rows 16*wave + NI*r + e, e < NI.
template <int D, int S>
struct Copier {
  uint32_t pk16;   // 16 * (pc ^ swz(16*wave + NI*r))
  int idx_off;     // first row of the lane inside a tile
  __device__ __forceinline__ void init(int wave, int lane) {
    const int r = lane / Geo<D>::CPR, pc = lane % Geo<D>::CPR;
    idx_off = 16 * wave + Geo<D>::NI * r;
    pk16 = 16u * (uint32_t)(pc ^ swz<D, S>(idx_off));
  }
  __device__ __forceinline__ uint32_t add(int e) const {
    return pk16 ^ (16u * (uint32_t)swz<D, S>(e));
  }
};

template <int D>
struct Idx {
  int v[Geo<D>::NI];
};

// Row indices of the lane's NI rows of tile `tile` of an index list.
template <int D>
__device__ __forceinline__ Idx<D> load_idx(const int32_t* idx, int tile, int idx_off) {
  Idx<D> r;
  const int32_t* p = idx + tile * kSlab + idx_off;
  if constexpr (Geo<D>::NI == 4) {
    const u32x4 w = *reinterpret_cast<const u32x4*>(p);
#pragma unroll
    for (int e = 0; e < 4; ++e) r.v[e] = (int)w[e];
  } else {
    const u32x2 w = *reinterpret_cast<const u32x2*>(p);
#pragma unroll
    for (int e = 0; e < 2; ++e) r.v[e] = (int)w[e];
  }
  return r;
}

// The copies address a row as row * row_stride_bytes with one 24 x 24-bit
// multiply: the entry points check this bound on the views they copy from
// (their 4 GiB span bound then keeps the product within 32 bits).
__host__ __device__ constexpr bool copy_rows_ok(int64_t rows, int64_t row_stride_elems) {
  return rows <= (1ll << 24) && row_stride_elems < (1ll << 23);
}

// The LDS DMA instructions are issued from inline assembly.  Issued through
// the compiler builtin, an LDS DMA in flight makes the compiler wait for *all*
// outstanding LDS reads (lgkmcnt(0)) before the first use of any of them, so a
// wave could never keep more than the reads of one MFMA in flight while its
// copies are pending -- which, with the copies overlapping the whole tile
// iteration, is always.  Hidden in assembly the copies are invisible to that
// bookkeeping; every copy is instead waited for explicitly (wait_copies, i.e.
// vmcnt(0), then a workgroup barrier) before any LDS read of its stage.  The
// LDS destination goes in M0 (set by the compiler through the "{m0}" operand;
// the leading s_nop is the wait state between an M0 write and its use).  The
// destination pointer must be wave-uniform.
__device__ __forceinline__ void dma16(const char* gbase, uint32_t voff, const char* lds) {
  const uint32_t l = (uint32_t)(uintptr_t)lds;
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :: "v"(voff), "s"(gbase), "{m0}"(l) : "memory");
}
__device__ __forceinline__ void dma4(const void* gbase, uint32_t voff, const char* lds) {
  const uint32_t l = (uint32_t)(uintptr_t)lds;
  asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, %1"
               :: "v"(voff), "s"(gbase), "{m0}"(l) : "memory");
}
// 4 bytes per lane from a per-lane 64-bit address.
__device__ __forceinline__ void dma4_lane(const void* gaddr, const char* lds) {
  const uint32_t l = (uint32_t)(uintptr_t)lds;
  asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, off"
               :: "v"(gaddr), "{m0}"(l) : "memory");
}

// Copy e of one tile: 16 bytes per lane, 1 KB per wave instruction.  g points
// at the head's first element of row 0 of the source tensor; rows are
// addressed with 32-bit byte offsets (scalar base + 32-bit vector offset).
template <int D, int S>
__device__ __forceinline__ void copy_one(const char* g, uint32_t ss_bytes, const Copier<D, S>& cp,
                                         const Idx<D>& ix, int e, char* slot, int wave) {
  const uint32_t off = __umul24((uint32_t)ix.v[e], ss_bytes) + cp.add(e);
  dma16(g, off, slot + (16 * wave + Geo<D>::NR * e) * Geo<D>::ROWB);
}

template <int D, int S>
__device__ __forceinline__ void copy_tile(const char* g, uint32_t ss_bytes, const Copier<D, S>& cp,
                                          const Idx<D>& ix, char* slot, int wave) {
#pragma unroll
  for (int e = 0; e < Geo<D>::NI; ++e) copy_one<D, S>(g, ss_bytes, cp, ix, e, slot, wave);
}

// One dword per row of a tile (masks, per-row scalars), natural row order.
__device__ __forceinline__ void copy_dwords(const void* m, char* slot, int lane) {
  dma4(m, 4u * (uint32_t)lane, slot);
}

__device__ __forceinline__ void wait_copies() {
  __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0), other counters untouched
}

// ---- MFMA operand reads ------------------------------------------------------

// Row operand of v_mfma_f32_32x32x16_bf16 from a tile: lane l holds row
// (rb*32 + l%32), elements 16c + 8*(l/32) .. +8.  Offsets are tile-relative.
template <int D, int S>
__device__ __forceinline__ int row_read_off(int lane, int c) {
  const int rr = lane & 31;
  return prow<D>(rr) * Geo<D>::ROWB + 16 * (((lane >> 5) + 2 * c) ^ swz<D, S>(rr));
}

// Transposed operand: lane l (group g = l/16, i = l%16) reads 4 elements of
// column block d0 = 32*db + 16*((l>>4)&1), rows 16kc + 4*(l>>5) + (i>>2) (lo)
// and +8 (hi); after ds_read_b64_tr_b16 lane l holds column d0 + i of those
// 4 + 4 rows.  Returns the tile-relative offset of the lo (hi = 1) read for
// row chunk kc = 0; chunk kc adds 16*kc rows.
template <int D, int S>
__device__ __forceinline__ int tr_read_off(int lane, int db, int hi) {
  const int i = lane & 15;
  const int row = 4 * (lane >> 5) + (i >> 2) + 8 * hi;
  const int q = 2 * ((lane >> 4) & 1) + ((i & 3) >> 1);
  return prow<D>(row) * Geo<D>::ROWB + 16 * ((4 * db + q) ^ swz<D, S>(row)) + 8 * (i & 1);
}

__device__ __forceinline__ bf16x8 tr_read(const char* lo, const char* hi) {
  const s16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)lo);
  const s16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)hi);
  return __builtin_bit_cast(bf16x8, __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7));
}

__device__ __forceinline__ f32x16 mfma(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

}  // namespace tile
}  // namespace hier
