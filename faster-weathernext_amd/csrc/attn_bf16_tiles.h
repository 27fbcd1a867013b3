// bfloat16 tile helpers shared by the bf16 kernels and the split-precision (bf16x3) forward: the
// LDS tile layout (row-major [rows][D], 16-byte chunks XOR-swizzled), its copies by the buffer
// unit's LDS DMA, and the per-lane offsets of the MFMA operand reads (row reads, ds_read_b64_tr_b16
// transpose reads).
#pragma once

#include "attn_device.h"

namespace fwn {
namespace {

using namespace dev;

// XOR swizzle of the 16-byte chunk index of a bf16 row-major tile with C chunks per row; depends
// on the row's low 4 bits only. Over the 16 rows of a row read it is a bijection within each set of
// rows that share a 256-byte bank line (row reads), and it sends the aligned 4-chunk group of each
// of 4 consecutive rows to a distinct part of the bank line (transpose reads).
template <int C>
__device__ __forceinline__ int swz(int row) {
  if constexpr (C >= 16) {
    return ((row & 3) << 2) | ((row >> 2) & 3);
  } else if constexpr (C == 8) {
    return (((row >> 1) & 1) << 2) | ((row >> 2) & 3);
  } else {
    return (row >> 2) & 3;
  }
}

// The swizzle of the 16-key dK/dV kernel's Q and dO tiles. gfx950 serves a ds_read_b128 in four
// 16-lane groups {l, l + 32 : l in [8k, 8k + 8)} and a ds_read_b64_tr_b16 in two 32-lane halves
// (measured with bank-conflict counters). In this kernel's row reads, each b128 group covers 8
// aligned rows at two logical chunks x and x ^ 2; in its transpose reads, each half covers 8
// aligned rows x one chunk pair (32 bytes). Over any 8 aligned rows, s(row) must therefore keep
// bits {0, 2, 3} distinct (row reads) and bits {1, 2, 3} distinct (transpose reads), per row
// position within a 256-byte bank line when a line holds 2 or 4 rows: s = (hi << 2) | 3 lo, with
// lo one row bit and hi the row bits above it. Depends on the row's low 3 bits only.
template <int C>
__device__ __forceinline__ int swz16(int row) {
  constexpr int sh = C >= 16 ? 0 : (C == 8 ? 1 : 2);
  return (((row & 7) >> (sh + 1)) << 2) | (((row >> sh) & 1) * 3);
}

template <int C, bool K16>
__device__ __forceinline__ int tile_swz(int row) {
  if constexpr (K16) {
    return swz16<C>(row);
  } else {
    return swz<C>(row);
  }
}

template <int D>
struct Tile {
  static constexpr int C = D / 8;                     // 16-byte chunks per row
  static constexpr int BYTES = BLK * D * 2;           // one 128 x D tile
  static constexpr int ROWS_PER_OP = 64 / C;          // rows one wave-wide DMA instruction fills
  static constexpr int OPS_PER_WAVE = BLK / ROWS_PER_OP / 4;
};

// Global -> LDS copy of one 128 x D tile by the 4 waves (buffer_load_dwordx4 ... lds).
// Instruction (op, w) fills physical chunks [(4*op + w) * 64, +64): lane l the chunk at row
// (4*op + w) * ROWS_PER_OP + l / C, physical column l % C, which holds logical column
// (l % C) ^ swz(row). The swizzle depends on row % 16, which is the same for every op.
template <int D, bool K16 = false>
struct TileDma {
  static constexpr int C = Tile<D>::C;
  static constexpr int RPO = Tile<D>::ROWS_PER_OP;
  uint32_t voff;

  __device__ __forceinline__ void init(int w, int lane, uint32_t snb) {
    const int row = w * RPO + lane / C;
    voff = (uint32_t)row * snb + (uint32_t)((((lane % C) ^ tile_swz<C, K16>(row))) << 4);
  }

  // Copies the rows of the tile's 32-row groups in `live` (bit c: rows 32c..32c+31, a
  // wave-uniform set); the rows of the other groups keep stale data and must not be read.
  __device__ __forceinline__ void issue(rsrc_t r, lds_char* tile, int w, int row0, uint32_t snb,
                                        uint32_t live = 15u) const {
    // The LDS destinations are loop-invariant; left visible, the compiler keeps all of them in
    // SGPRs across the tile loop and spills other scalars. The empty asm makes the base opaque,
    // so each destination is one scalar add at the copy.
    uint32_t base = (uint32_t)(uintptr_t)tile + (uint32_t)w * 1024u;
    asm volatile("" : "+s"(base));
#pragma unroll
    for (int op = 0; op < Tile<D>::OPS_PER_WAVE; ++op) {
      if (!(live >> ((op * 4 * RPO + w * RPO) >> 5) & 1u)) continue;  // this op's rows lie in one group
      const uint32_t vo = voff + (uint32_t)(row0 + op * 4 * RPO) * snb;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)(uintptr_t)(base + op * 4096u),
                                               16, (int)vo, 0, 0, 0);
    }
  }
};

// Per-lane LDS byte offsets of the MFMA A operands.
//   row[s]:     sigma-ordered row of this lane, columns 16*s + 8*g.. (+ sb * 32 * 2D).
//   tr[db][h]:  transpose read for columns 32*db.. and keys 8*g + 4*h.. of a 16-key chunk
//               (+ (32*sb + 16*c) * 2D).
template <int D>
struct Off {
  static constexpr int C = Tile<D>::C;
  uint32_t row[D / 16];
  uint32_t tr[D / 32][2];

  __device__ __forceinline__ void init(int lane) {
    const int i = lane & 31, g = lane >> 5;
    const int rho = sigma(i);
#pragma unroll
    for (int s = 0; s < D / 16; ++s) row[s] = rho * (2 * D) + (((2 * s + g) ^ swz<C>(rho)) << 4);
    const int G = lane >> 4, t = lane & 15, e = t >> 2, q = t & 3, gg = G >> 1;
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int r = 8 * gg + 4 * h + e;
        const int chunk = 4 * db + 2 * (G & 1) + (q >> 1);
        tr[db][h] = r * (2 * D) + ((chunk ^ swz<C>(r)) << 4) + (q & 1) * 8;
      }
  }
};

__device__ __forceinline__ u32x4 row_read(const lds_char* tile, uint32_t off) {
  return *(const __attribute__((address_space(3))) u32x4*)(tile + off);
}

__device__ __forceinline__ u32x2 tr_read(const lds_char* tile, uint32_t off) {
  const i16x4 v =
      __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4*)(tile + off));
  return __builtin_bit_cast(u32x2, v);
}

// A operand of the second contraction for columns 32*db.. and keys 32*sb + 16*c .. +15.
template <int D>
__device__ __forceinline__ u32x4 tr_operand(const lds_char* tile, const Off<D>& off, int db, int sb, int c) {
  const uint32_t base = (uint32_t)(32 * sb + 16 * c) * (2 * D);
  const u32x2 lo = tr_read(tile, off.tr[db][0] + base), hi = tr_read(tile, off.tr[db][1] + base);
  return u32x4{lo[0], lo[1], hi[0], hi[1]};
}

// This lane's row fragment (B operand of the first contraction): columns 16*s + 8*g .. +7.
template <int D>
__device__ __forceinline__ void load_frag(u32x4 (&f)[D / 16], rsrc_t r, int row, uint32_t snb, int g) {
#pragma unroll
  for (int s = 0; s < D / 16; ++s) f[s] = bload16(r, (uint32_t)row * snb + (uint32_t)(32 * s + 16 * g));
}

}  // namespace
}  // namespace fwn
