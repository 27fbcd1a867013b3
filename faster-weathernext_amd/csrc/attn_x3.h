// Building blocks of the bf16x3 (split-precision) kernels: the hi/lo split of float32 values,
// the three-part product on V_MFMA_F32_32X32X16_BF16, split row fragments and the LDS DMA of
// split rows (four 32-row planes per step).
#pragma once

#include "attn_bf16_tiles.h"

namespace fwn {
namespace {

using namespace dev;

// hi = bf16(x) (round to nearest even), lo = bf16(x - hi): x - hi is exact in fp32.
__device__ __forceinline__ void split8(const float (&x)[8], u32x4& hi, u32x4& lo) {
  bf16x8 h, l;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    h[e] = (__bf16)x[e];
    l[e] = (__bf16)(x[e] - (float)h[e]);
  }
  hi = __builtin_bit_cast(u32x4, h);
  lo = __builtin_bit_cast(u32x4, l);
}

// Elements 8 * half .. + 7 of an accumulator, split.
__device__ __forceinline__ void split_acc(const f32x16& v, int half, u32x4& hi, u32x4& lo) {
  float x[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = v[8 * half + e];
  split8(x, hi, lo);
}

// The three-part product into c: the two cross terms first, then hi * hi.
__device__ __forceinline__ f32x16 mfma_x3(const u32x4& ah, const u32x4& al, const u32x4& bh, const u32x4& bl,
                                          f32x16 c) {
  c = mfma_bf16(al, bh, c);
  c = mfma_bf16(ah, bl, c);
  return mfma_bf16(ah, bh, c);
}

// This lane's row fragment of a float32 tensor (columns 16 s + 8 g .. + 7 of `row`), split: the B
// operands of the first contractions.
template <int D>
__device__ __forceinline__ void load_frag_x3(u32x4 (&hi)[D / 16], u32x4 (&lo)[D / 16], rsrc_t r, int row,
                                             uint32_t snb, int g) {
  const uint32_t off = (uint32_t)row * snb + (uint32_t)(32 * g);
#pragma unroll
  for (int s = 0; s < D / 16; ++s) {
    const f32x4 x0 = __builtin_bit_cast(f32x4, bload16(r, off + 64 * s));
    const f32x4 x1 = __builtin_bit_cast(f32x4, bload16(r, off + 64 * s + 16));
    const float x[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
    split8(x, hi[s], lo[s]);
  }
}

// Copy of 32 split rows of two operands (forward: K and V; dK/dV: Q and dO; dQ: two key groups of
// K) into a group buffer of four 32-row planes (A hi, A lo, B hi, B lo; each [32][D] bf16, chunks
// swizzled as the bf16 tiles). Each wave-wide
// LDS DMA instruction fills 1 KB = RPO rows of one plane; the 4 waves share the 4 * NI
// instructions of a step. Lane l of instruction (plane, sub) copies row RPO * sub + l / C,
// physical chunk l % C, which holds logical chunk (l % C) ^ swz(row); the swizzle depends on
// row % 16, which is the same for every instruction of one wave.
template <int D>
struct X3Dma {
  static constexpr int C = D / 8;
  static constexpr int RPO = 1024 / (2 * D);
  static constexpr int NI = 32 / RPO;
  static constexpr int GB = 32 * 2 * D;  // bytes of one plane
  static constexpr int XROW = 4 * D;     // bytes of one split row (hi, lo)
  uint32_t voff;

  __device__ __forceinline__ void init(int w, int lane) {
    const int row = RPO * (w % NI) + lane / C;
    voff = (uint32_t)(lane / C) * XROW + (uint32_t)(((lane % C) ^ swz<C>(row)) << 4);
  }

  // Planes 0, 1 from rA (rows row0 .. row0 + 31, hi and lo), planes 2, 3 from rB; only the planes
  // in `planes` (bit p: plane p, a wave-uniform set) are copied.
  __device__ __forceinline__ void issue(rsrc_t rA, rsrc_t rB, lds_char* buf, int row0, int w,
                                        uint32_t planes = 15u) const {
    uint32_t base = (uint32_t)(uintptr_t)buf;
    asm volatile("" : "+s"(base));
#pragma unroll
    for (int m = 0; m < D / 16; ++m) {
      int plane, sub;
      if constexpr (NI >= 4) {
        plane = 4 * m / NI;
        sub = w + (4 * m) % NI;
      } else {
        plane = 2 * m + (w >> 1);
        sub = w & 1;
      }
      if (!(planes >> plane & 1u)) continue;
      const uint32_t src = (uint32_t)(row0 + RPO * sub) * XROW + voff + (uint32_t)(plane & 1) * (2 * D);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          m < D / 32 ? rA : rB,
          (__attribute__((address_space(3))) void*)(uintptr_t)(base + (uint32_t)(plane * GB + sub * 1024)), 16,
          (int)src, 0, 0, 0);
    }
  }
};

constexpr int kNonTemporal = 2;  // buffer load/store cache policy: non-temporal (gfx950 "nt")
constexpr uint32_t kPastEnd = 0x7FFFFFF0u;  // a buffer offset past every slice: reads zeros

}  // namespace

// dK/dV of the bf16x3 backward with the dS exchange (attn_x3_dkv.hip).
hipError_t launch_x3_dkv(int head_dim, const KArgs& a, hipStream_t stream);

}  // namespace fwn
