// Block-sparse masked flash attention for gfx950 (MI355X): forward, dQ, dK/dV, delta.
//
// One workgroup = 4 waves = one 128-row block of queries (forward, dQ) or keys (dK/dV) for one
// (batch, head); each wave owns 32 rows. The workgroup walks the block's live 128x128 tiles
// (CSR list), stages the tile's operands in LDS and runs both contractions on MFMA:
//   bf16: V_MFMA_F32_32X32X16_BF16 (fp32 accumulate), fp32: V_MFMA_F32_32X32X2_F32.
//
// Layout shared by every kernel. The first contraction is computed transposed,
// X^T[col][row] (e.g. S^T = K Q^T in the forward), so the accumulator column (lane % 32) is the
// wave's own row (query) and the softmax statistics are per lane. The operand rows of that MFMA
// are loaded in the permuted order sigma(), which makes accumulator register r of lane group g
// hold column 16*(r/8) + 8*g + r%8 of each 32-column sub-block: 8 consecutive columns per lane
// group and 16-column chunk. That is exactly the B-operand layout of the second contraction
// (O^T += V^T P^T), so P (and dS) go from accumulator to MFMA operand in registers, with one
// fp32->bf16 pack, and never touch LDS. The second contraction's A operand (V^T, K^T, Q^T, dO^T)
// needs the contracted column contiguous per lane: bf16 tiles are transposed once while being
// staged (8x8 register transpose), fp32 operands are one element per lane and are read straight
// from the row-major tile.
//
// Global memory is accessed through raw buffer resources, one per (batch, head) slice, whose
// hardware range check returns zeros for rows >= n and drops their stores, so ragged blocks
// need no branches.
//
// Masking: the tile's bitmask is prepared on the host as one 64-bit lane mask per accumulator
// element (fwn_tiles_prepare), read with scalar loads and applied with one v_cndmask per element
// (skipped for fully valid tiles). Masked logits are -inf; a row with no valid key so far uses 0
// as its exponent base, so masked entries contribute exactly 0 and nothing becomes NaN. Every
// real row attends to at least itself in a k-hop mask; rows without any valid key produce 0.
//
// Reference: pallas_attn.py:112-141 (forward), 161-215 (dQ, dK/dV), 274-311 (VJP driver).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "attn_kernels.h"

namespace fwn {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __amdgpu_buffer_rsrc_t rsrc_t;

// Uniform metadata (tile list, lane masks) is read through the constant address space so the
// compiler uses scalar loads into SGPRs.
typedef const __attribute__((address_space(4))) uint64_t* cu64_ptr;
typedef const __attribute__((address_space(4))) uint32_t* cu32_ptr;
typedef const __attribute__((address_space(4))) int32_t* ci32_ptr;

constexpr int BLK = 128;
constexpr int NT = 256;
constexpr int RSRC_DW3 = 0x00020000;  // raw buffer, 32-bit dword format (gfx9 family)
constexpr float LOG2E = 1.4426950408889634f;
constexpr float LN2 = 0.6931471805599453f;

// ------------------------------------------------------------------------------------------
// Small helpers.

// Operand row that MFMA row i of a 32-row sub-block loads (see the file comment).
__device__ __forceinline__ int sigma(int i) {
  return ((i >> 4) << 4) | (((i >> 2) & 1) << 3) | (((i >> 3) & 1) << 2) | (i & 3);
}

// Column (key / query) within a 128-wide tile held by accumulator register r of sub-block sb.
__device__ __forceinline__ int element_col(int sb, int r, int g) {
  return 32 * sb + 16 * (r >> 3) + 8 * g + (r & 7);
}

// XOR swizzle of the 16-byte chunk index of row-major tiles with C chunks per row, chosen so the
// sigma-ordered operand reads (rows 0-3, 8-11, 4-7, 12-15 in lanes 0-15) and the staging writes
// hit distinct banks. Depends on the row's low 4 bits only.
template <int C>
__device__ __forceinline__ int swz_row(int row) {
  if constexpr (C == 4) {
    return (((row >> 1) ^ (row >> 2)) & 1) | (((row >> 3) & 1) << 1);
  } else if constexpr (C == 8) {
    return ((row ^ (row >> 2)) & 1) | (((row >> 1) & 1) << 1) | (((row >> 3) & 1) << 2);
  } else {
    return (row & 3) | (((row >> 3) & 1) << 2) | (((row >> 2) & 1) << 3);
  }
}

// 3-bit variant for fp32 tiles: keeps 32-column blocks of a row inside one aligned 128 bytes.
__device__ __forceinline__ int swz_row3(int row) { return (row & 3) | (((row >> 3) & 1) << 2); }

// Swizzle of transposed bf16 tiles ([D][128], 16 chunks per row); depends on d mod 32 only, so
// the per-lane read offsets of all 32-row blocks differ by immediates.
__device__ __forceinline__ int swz_t(int d) { return (d & 15) ^ (((d >> 3) & 3) << 1); }

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, RSRC_DW3);
}

__device__ __forceinline__ u32x4 bload16(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
}

__device__ __forceinline__ u32x4 lds16(const char* p) { return *(const u32x4*)p; }

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int r = 0; r < 16; ++r) z[r] = 0.f;
  return z;
}

// Bit `lane` of the wave-uniform mask `sel` ? x : y. inverse_ballot turns the 64-bit SGPR mask
// into the per-lane condition, so this is one v_cndmask with the SGPR pair as its selector, and
// (unlike inline assembly) the compiler sees the operands and inserts the wait states an MFMA
// result needs before a VALU read.
__device__ __forceinline__ float select_lane(uint64_t sel, float x, float y) {
  return __builtin_amdgcn_inverse_ballot_w64(sel) ? x : y;
}

// 2^x on the hardware transcendental unit (V_EXP_F32); callers fold log2(e) into their scales.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ bf16x8 pack_bf16(const f32x16& v, int half) {
  bf16x8 r;
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = (__bf16)v[8 * half + e];
  return r;
}

__device__ __forceinline__ f32x16 mfma_bf16(const u32x4& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x16 mfma_bf16(const u32x4& a, const u32x4& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                 c, 0, 0, 0);
}

__device__ __forceinline__ f32x16 mfma_f32(float a, float b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// Transposes an 8x8 block of bf16 (8 rows of 16 bytes) in registers: y[c] = column c.
__device__ __forceinline__ void transpose8x8(const u32x4 (&x)[8], u32x4 (&y)[8]) {
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const int word = c >> 1;
    const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;
#pragma unroll
    for (int e = 0; e < 4; ++e) y[c][e] = __builtin_amdgcn_perm(x[2 * e + 1][word], x[2 * e][word], sel);
  }
}

struct Job {
  int blk;
  int b, h;
  int64_t base;  // element offset of (b, h)
};

// Blocks are visited in `order` (most tiles first); the (batch, head) index varies fastest, so
// the heads of one block run side by side and share its mask words in L2.
__device__ __forceinline__ Job decode_job(const KArgs& a) {
  Job j;
  const int bh_count = a.batch * a.heads;
  const int slot = blockIdx.x / bh_count;
  const int bh = blockIdx.x - slot * bh_count;
  j.blk = a.order ? ((ci32_ptr)a.order)[slot] : slot;
  j.b = bh / a.heads;
  j.h = bh - j.b * a.heads;
  j.base = (int64_t)j.b * a.sb + (int64_t)j.h * a.sh;
  return j;
}

__device__ __forceinline__ void tile_range(const KArgs& a, int blk, int& t0, int& t1) {
  t0 = ((ci32_ptr)a.ptr)[blk];
  t1 = ((ci32_ptr)a.ptr)[blk + 1];
  t0 = t0 < 0 ? 0 : t0;
  t1 = t1 > a.n_tiles ? a.n_tiles : t1;
}

__device__ __forceinline__ int64_t stat_index(const KArgs& a, const Job& j, int row) {
  return ((int64_t)j.b * a.heads + j.h) * a.n + row;
}

// ------------------------------------------------------------------------------------------
// bf16 staging. The first D/32 waves stage a 128 x D tile; lane -> (column chunk dc, row block
// kblk) = (4*wave + lane % 4, lane / 4), so each lane owns an 8-row x 8-column block: lanes
// 0-3 read 64 contiguous bytes of a row. The block is written row-major (swizzled) and/or
// transposed (8x8 register transpose) into LDS.

template <int D>
struct Bf16Stage {
  static constexpr int C = D / 8;
  static constexpr int WAVES = C / 4;
  u32x4 x[8];
  uint32_t voff;  // byte offset of (row 8*kblk, chunk dc) in the (batch, head) slice
  int dc, kblk;

  __device__ __forceinline__ static bool active(int wave) { return wave < WAVES; }

  __device__ __forceinline__ void init(int wave, int lane, uint32_t snb) {
    dc = 4 * wave + (lane & 3);
    kblk = lane >> 2;
    voff = (uint32_t)(8 * kblk) * snb + (uint32_t)(16 * dc);
  }

  __device__ __forceinline__ void load(rsrc_t r, int row0, uint32_t snb) {
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = bload16(r, voff + (uint32_t)(row0 + e) * snb);
  }

  // The store addresses are recomputed at every call (the empty asm hides that dc and kblk are
  // loop-invariant): keeping 16 hoisted addresses alive across the tile loop costs more VGPRs than
  // the few VALU ops it saves.
  __device__ __forceinline__ void store_rows(char* lds) const {
    int dcv = dc, kb = kblk;
    asm volatile("" : "+v"(dcv), "+v"(kb));
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int row = 8 * kb + e;
      *(u32x4*)(lds + row * (D * 2) + ((dcv ^ swz_row<C>(row)) << 4)) = x[e];
    }
  }

  __device__ __forceinline__ void store_transposed(char* lds) const {
    int dcv = dc, kb = kblk;
    asm volatile("" : "+v"(dcv), "+v"(kb));
    u32x4 y[8];
    transpose8x8(x, y);
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const int d = 8 * dcv + c;
      *(u32x4*)(lds + d * 256 + ((kb ^ swz_t(d)) << 4)) = y[c];
    }
  }
};

// Per-lane LDS offsets of the MFMA A operands (bf16).
template <int D>
struct Bf16Offsets {
  uint32_t row[D / 16];  // row-major tile, sigma row of this lane, step s: + sb * 32 * 2D
  uint32_t tr[8];        // transposed tile, row i, chunk 4*sb + 2*c + g: + db * 32 * 256

  __device__ __forceinline__ void init(int i, int g) {
    constexpr int C = D / 8;
    const int rho = sigma(i);
#pragma unroll
    for (int s = 0; s < D / 16; ++s) row[s] = rho * (D * 2) + (((2 * s + g) ^ swz_row<C>(rho)) << 4);
#pragma unroll
    for (int k = 0; k < 8; ++k) tr[k] = i * 256 + (((2 * k + g) ^ swz_t(i)) << 4);
  }
};

// This lane's row fragment: row `row`, columns 16*s + 8*g .. +7 for each MFMA step s.
template <int D>
__device__ __forceinline__ void load_frag_bf16(u32x4 (&f)[D / 16], rsrc_t r, int row, uint32_t snb, int g) {
#pragma unroll
  for (int s = 0; s < D / 16; ++s) f[s] = bload16(r, (uint32_t)row * snb + (uint32_t)(32 * s + 16 * g));
}

// Stores a transposed accumulator (rows d, column = this lane's row) as bf16, times `mul`.
template <int D>
__device__ __forceinline__ void store_acc_bf16(rsrc_t r, int row, uint32_t snb, const f32x16 (&acc)[D / 32],
                                               float mul, int g) {
#pragma unroll
  for (int db = 0; db < D / 32; ++db) {
#pragma unroll
    for (int k4 = 0; k4 < 4; ++k4) {
      const int d = 32 * db + 8 * k4 + 4 * g;
      u32x2 w;
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) {
        const __bf16 lo = (__bf16)(acc[db][4 * k4 + 2 * h2] * mul);
        const __bf16 hi = (__bf16)(acc[db][4 * k4 + 2 * h2 + 1] * mul);
        w[h2] = (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
      }
      __builtin_amdgcn_raw_buffer_store_b64(w, r, (int)((uint32_t)row * snb + (uint32_t)(2 * d)), 0, 0);
    }
  }
}

// ------------------------------------------------------------------------------------------
// fp32 staging: linear chunk mapping (coalesced), row-major tiles in LDS, optionally swizzled.

template <int D>
__device__ __forceinline__ void stage_rows_f32(char* lds, rsrc_t r, int row0, uint32_t snb, int tid, bool swizzle) {
  constexpr int C = D / 4;
  constexpr int PER = BLK * C / NT;
#pragma unroll
  for (int it = 0; it < PER; ++it) {
    const int id = tid + it * NT;
    const int row = id / C, ch = id % C;
    const u32x4 x = bload16(r, (uint32_t)(row0 + row) * snb + (uint32_t)(16 * ch));
    const int pc = swizzle ? (ch ^ swz_row3(row)) : ch;
    *(u32x4*)(lds + row * (D * 4) + (pc << 4)) = x;
  }
}

// Per-lane LDS offsets of the fp32 MFMA A operands.
//   row[u & 3]: sigma row of this lane, chunk 2*u + g of a swizzled tile;
//               + 128 * (u / 4) + sb * 32 * 4D.
//   el[r & 3]:  element (row element_col(sb, r, g), column 32*db + i) of a swizzled tile;
//               + (32*sb + 16*(r/8) + r%8) * 4D + 128 * db.
//   el_plain:   the same element of an unswizzled tile.
template <int D>
struct F32Offsets {
  uint32_t row[4];
  uint32_t el[4];
  uint32_t el_plain;

  __device__ __forceinline__ void init(int i, int g) {
    const int rho = sigma(i);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      row[k] = rho * (D * 4) + ((((2 * k + g) & 7) ^ swz_row3(rho)) << 4);
      el[k] = 8 * g * (D * 4) + ((((i >> 2) ^ (k | (g << 2)))) << 4) + ((i & 3) << 2);
    }
    el_plain = 8 * g * (D * 4) + 4 * i;
  }
  __device__ __forceinline__ static uint32_t row_imm(int sb, int u) { return sb * 32 * (D * 4) + 128 * (u >> 2); }
  __device__ __forceinline__ static uint32_t el_imm(int sb, int r, int db) {
    return (32 * sb + 16 * (r >> 3) + (r & 7)) * (D * 4) + 128 * db;
  }
};

// fp32 fragment: f[u] = columns 8*u + 4*g .. +3 of `row` (MFMA step 4*u + e uses f[u][e]).
template <int D>
__device__ __forceinline__ void load_frag_f32(f32x4 (&f)[D / 8], rsrc_t r, int row, uint32_t snb, int g) {
#pragma unroll
  for (int u = 0; u < D / 8; ++u)
    f[u] = __builtin_bit_cast(f32x4, bload16(r, (uint32_t)row * snb + (uint32_t)(32 * u + 16 * g)));
}

template <int D>
__device__ __forceinline__ void store_acc_f32(rsrc_t r, int row, uint32_t snb, const f32x16 (&acc)[D / 32], float mul,
                                              int g) {
#pragma unroll
  for (int db = 0; db < D / 32; ++db) {
#pragma unroll
    for (int k4 = 0; k4 < 4; ++k4) {
      const int d = 32 * db + 8 * k4 + 4 * g;
      f32x4 w;
#pragma unroll
      for (int e = 0; e < 4; ++e) w[e] = acc[db][4 * k4 + e] * mul;
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, w), r,
                                             (int)((uint32_t)row * snb + (uint32_t)(4 * d)), 0, 0);
    }
  }
}

// ------------------------------------------------------------------------------------------
// Online softmax step of the forward kernels. s[sb][r] holds this lane's logits (raw q.k) of
// the tile; on return it holds the unnormalised probabilities exp2(s*c2 - m).

struct SoftmaxState {
  float m;  // running max of s*c2 (log2 domain), -inf before the first valid key
  float l;  // running sum of exp2(s*c2 - m) over this lane's half of the keys
};

__device__ __forceinline__ float softmax_tile(f32x16 (&s)[4], SoftmaxState& st, float c2) {
  const float ninf = -__builtin_inff();
  float mx = s[0][0];
#pragma unroll
  for (int sb = 0; sb < 4; ++sb)
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[sb][r]);
  mx = fmaxf(mx, __shfl_xor(mx, 32));
  const float m_new = fmaxf(st.m, mx * c2);
  const float base = m_new == ninf ? 0.f : m_new;
  const float corr = fast_exp2(st.m - base);
  float sum = 0.f;
#pragma unroll
  for (int sb = 0; sb < 4; ++sb)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float p = fast_exp2(fmaf(s[sb][r], c2, -base));
      s[sb][r] = p;
      sum += p;
    }
  st.l = st.l * corr + sum;
  st.m = m_new;
  return corr;
}

// The 16 lane masks of sub-block sb of a tile (scalar loads, issued ahead of the sub-block's MFMAs).
// Fully valid tiles hold all-ones words, so masks are applied unconditionally: one v_cndmask per
// element and no branch.
struct SubMask {
  uint64_t w[16];
  __device__ __forceinline__ void load(cu64_ptr mk, int sb) {
#pragma unroll
    for (int r = 0; r < 16; ++r) w[r] = mk[sb * 16 + r];
  }
};

// Natural log-sum-exp of the scaled logits: (m + log2 l) * ln 2 (pallas_attn.py:140-141).
__device__ __forceinline__ void write_lse(const KArgs& a, const Job& j, int row, const SoftmaxState& st, float ltot) {
  if (a.lse_out && row < a.n) {
    const float lse = (st.m + __builtin_amdgcn_logf(fmaxf(ltot, 1e-30f))) * LN2;
    a.lse_out[stat_index(a, j, row)] = lse;
  }
}

// ------------------------------------------------------------------------------------------
// Forward, bf16. 64 KB of LDS: two workgroups per CU.

template <int D>
__global__ void __launch_bounds__(NT, 2) fwd_bf16_kernel(KArgs a) {
  __shared__ __attribute__((aligned(16))) char smem[2 * BLK * D * 2];
  char* ldsK = smem;                 // [128][D] row-major, swizzled
  char* ldsVt = smem + BLK * D * 2;  // [D][128] transposed
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i = lane & 31, g = lane >> 5;
  const Job j = decode_job(a);
  const uint32_t snb = (uint32_t)a.sn * 2;
  const rsrc_t rQ = make_rsrc((const uint16_t*)a.q + j.base, a.slice_bytes);
  const rsrc_t rK = make_rsrc((const uint16_t*)a.k + j.base, a.slice_bytes);
  const rsrc_t rV = make_rsrc((const uint16_t*)a.v + j.base, a.slice_bytes);

  const int qrow = j.blk * BLK + 32 * w + i;
  u32x4 qf[D / 16];
  load_frag_bf16<D>(qf, rQ, qrow, snb, g);
  Bf16Offsets<D> off;
  off.init(i, g);
  f32x16 o[D / 32];
#pragma unroll
  for (int db = 0; db < D / 32; ++db) o[db] = zero16();
  SoftmaxState st{-__builtin_inff(), 0.f};

  int t0, t1;
  tile_range(a, j.blk, t0, t1);
  Bf16Stage<D> ks, vs;
  const bool stager = Bf16Stage<D>::active(w);
  ks.init(w, lane, snb);
  vs.init(w, lane, snb);
  // K and V are loaded after the barrier that ends the previous tile's LDS reads, so the loaded
  // registers live only until their LDS store and the kernel stays within 256 VGPRs; with two
  // workgroups per CU the other workgroup computes while this one waits for memory.
  for (int tt = t0; tt < t1; ++tt) {
    const int t = __builtin_amdgcn_readfirstlane(tt);  // uniform: keeps tile metadata in SGPRs
    __syncthreads();
    if (stager) {
      const int kb = ((ci32_ptr)a.col)[t];
      ks.load(rK, kb * BLK, snb);
      vs.load(rV, kb * BLK, snb);
      ks.store_rows(ldsK);
      vs.store_transposed(ldsVt);
    }
    __syncthreads();
    const cu64_ptr mk = (cu64_ptr)a.lanes + ((int64_t)t * 4 + w) * 64;
    f32x16 s[4];
#pragma unroll
    for (int sb = 0; sb < 4; ++sb) {
      SubMask m;
      m.load(mk, sb);
      s[sb] = zero16();
#pragma unroll
      for (int step = 0; step < D / 16; ++step)
        s[sb] = mfma_bf16(lds16(ldsK + off.row[step] + sb * 32 * (D * 2)), qf[step], s[sb]);
#pragma unroll
      for (int r = 0; r < 16; ++r) s[sb][r] = select_lane(m.w[r], s[sb][r], -__builtin_inff());
    }
    const float corr = softmax_tile(s, st, a.c2);
#pragma unroll
    for (int db = 0; db < D / 32; ++db) o[db] *= corr;
#pragma unroll
    for (int sb = 0; sb < 4; ++sb) {
      const bf16x8 p0 = pack_bf16(s[sb], 0), p1 = pack_bf16(s[sb], 1);
#pragma unroll
      for (int db = 0; db < D / 32; ++db) {
        o[db] = mfma_bf16(lds16(ldsVt + off.tr[2 * sb] + db * 32 * 256), p0, o[db]);
        o[db] = mfma_bf16(lds16(ldsVt + off.tr[2 * sb + 1] + db * 32 * 256), p1, o[db]);
      }
    }
  }
  const float ltot = st.l + __shfl_xor(st.l, 32);
  const float inv = ltot > 0.f ? 1.f / ltot : 0.f;
  store_acc_bf16<D>(make_rsrc((uint16_t*)a.out0 + j.base, a.slice_bytes), qrow, snb, o, inv, g);
  if (g == 0) write_lse(a, j, qrow, st, ltot);
}

// ------------------------------------------------------------------------------------------
// Forward, fp32. 128 KB of LDS: one workgroup per CU.

template <int D>
__global__ void __launch_bounds__(NT, 1) fwd_f32_kernel(KArgs a) {
  __shared__ __attribute__((aligned(16))) char smem[2 * BLK * D * 4];
  char* ldsK = smem;                // [128][D] swizzled
  char* ldsV = smem + BLK * D * 4;  // [128][D] plain
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i = lane & 31, g = lane >> 5;
  const Job j = decode_job(a);
  const uint32_t snb = (uint32_t)a.sn * 4;
  const rsrc_t rQ = make_rsrc((const float*)a.q + j.base, a.slice_bytes);
  const rsrc_t rK = make_rsrc((const float*)a.k + j.base, a.slice_bytes);
  const rsrc_t rV = make_rsrc((const float*)a.v + j.base, a.slice_bytes);

  const int qrow = j.blk * BLK + 32 * w + i;
  f32x4 qf[D / 8];
  load_frag_f32<D>(qf, rQ, qrow, snb, g);
  F32Offsets<D> off;
  off.init(i, g);
  f32x16 o[D / 32];
#pragma unroll
  for (int db = 0; db < D / 32; ++db) o[db] = zero16();
  SoftmaxState st{-__builtin_inff(), 0.f};

  int t0, t1;
  tile_range(a, j.blk, t0, t1);
  for (int tt = t0; tt < t1; ++tt) {
    const int t = __builtin_amdgcn_readfirstlane(tt);
    const int kb = ((ci32_ptr)a.col)[t];
    __syncthreads();
    stage_rows_f32<D>(ldsK, rK, kb * BLK, snb, tid, true);
    stage_rows_f32<D>(ldsV, rV, kb * BLK, snb, tid, false);
    __syncthreads();
    const cu64_ptr mk = (cu64_ptr)a.lanes + ((int64_t)t * 4 + w) * 64;
    f32x16 s[4];
#pragma unroll
    for (int sb = 0; sb < 4; ++sb) {
      SubMask m;
      m.load(mk, sb);
      s[sb] = zero16();
#pragma unroll
      for (int u = 0; u < D / 8; ++u) {
        const f32x4 kx = *(const f32x4*)(ldsK + off.row[u & 3] + off.row_imm(sb, u));
#pragma unroll
        for (int e = 0; e < 4; ++e) s[sb] = mfma_f32(kx[e], qf[u][e], s[sb]);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) s[sb][r] = select_lane(m.w[r], s[sb][r], -__builtin_inff());
    }
    const float corr = softmax_tile(s, st, a.c2);
#pragma unroll
    for (int db = 0; db < D / 32; ++db) o[db] *= corr;
#pragma unroll
    for (int sb = 0; sb < 4; ++sb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
#pragma unroll
        for (int db = 0; db < D / 32; ++db)
          o[db] = mfma_f32(*(const float*)(ldsV + off.el_plain + off.el_imm(sb, r, db)), s[sb][r], o[db]);
      }
  }
  const float ltot = st.l + __shfl_xor(st.l, 32);
  const float inv = ltot > 0.f ? 1.f / ltot : 0.f;
  store_acc_f32<D>(make_rsrc((float*)a.out0 + j.base, a.slice_bytes), qrow, snb, o, inv, g);
  if (g == 0) write_lse(a, j, qrow, st, ltot);
}

// ------------------------------------------------------------------------------------------
// dQ, bf16: per query block over the forward tile list (pallas_attn.py:161-184).
// P = where(valid, exp(s*scale - lse), 0); dS = P * (dP - delta); dQ = scale * dS K.

template <int D>
__global__ void __launch_bounds__(NT, 1) dq_bf16_kernel(KArgs a) {
  __shared__ __attribute__((aligned(16))) char smem[3 * BLK * D * 2];
  char* ldsK = smem;                    // [128][D] swizzled
  char* ldsKt = smem + BLK * D * 2;     // [D][128]
  char* ldsV = smem + 2 * BLK * D * 2;  // [128][D] swizzled
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i = lane & 31, g = lane >> 5;
  const Job j = decode_job(a);
  const uint32_t snb = (uint32_t)a.sn * 2;
  const rsrc_t rK = make_rsrc((const uint16_t*)a.k + j.base, a.slice_bytes);
  const rsrc_t rV = make_rsrc((const uint16_t*)a.v + j.base, a.slice_bytes);

  const int qrow = j.blk * BLK + 32 * w + i;
  u32x4 qf[D / 16], df[D / 16];
  load_frag_bf16<D>(qf, make_rsrc((const uint16_t*)a.q + j.base, a.slice_bytes), qrow, snb, g);
  load_frag_bf16<D>(df, make_rsrc((const uint16_t*)a.dout + j.base, a.slice_bytes), qrow, snb, g);
  float lse_t = 0.f, delta = 0.f;
  if (qrow < a.n) {
    lse_t = a.lse[stat_index(a, j, qrow)] * LOG2E;
    delta = a.delta[stat_index(a, j, qrow)];
  }
  Bf16Offsets<D> off;
  off.init(i, g);
  f32x16 acc[D / 32];
#pragma unroll
  for (int db = 0; db < D / 32; ++db) acc[db] = zero16();

  int t0, t1;
  tile_range(a, j.blk, t0, t1);
  Bf16Stage<D> ks, vs;
  const bool stager = Bf16Stage<D>::active(w);
  ks.init(w, lane, snb);
  vs.init(w, lane, snb);
  if (t0 < t1 && stager) {
    const int kb = ((ci32_ptr)a.col)[t0];
    ks.load(rK, kb * BLK, snb);
    vs.load(rV, kb * BLK, snb);
  }
  for (int tt = t0; tt < t1; ++tt) {
    const int t = __builtin_amdgcn_readfirstlane(tt);
    __syncthreads();
    if (stager) {
      ks.store_rows(ldsK);
      ks.store_transposed(ldsKt);
      vs.store_rows(ldsV);
    }
    __syncthreads();
    if (t + 1 < t1 && stager) {
      const int kb = ((ci32_ptr)a.col)[t + 1];
      ks.load(rK, kb * BLK, snb);
      vs.load(rV, kb * BLK, snb);
    }
    const cu64_ptr mk = (cu64_ptr)a.lanes + ((int64_t)t * 4 + w) * 64;
#pragma unroll
    for (int sb = 0; sb < 4; ++sb) {
      SubMask m;
      m.load(mk, sb);
      f32x16 s = zero16(), dp = zero16();
#pragma unroll
      for (int step = 0; step < D / 16; ++step) {
        s = mfma_bf16(lds16(ldsK + off.row[step] + sb * 32 * (D * 2)), qf[step], s);
        dp = mfma_bf16(lds16(ldsV + off.row[step] + sb * 32 * (D * 2)), df[step], dp);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float p = fast_exp2(fmaf(s[r], a.c2, -lse_t));
        p = select_lane(m.w[r], p, 0.f);
        dp[r] = p * (dp[r] - delta);
      }
      const bf16x8 d0 = pack_bf16(dp, 0), d1 = pack_bf16(dp, 1);
#pragma unroll
      for (int db = 0; db < D / 32; ++db) {
        acc[db] = mfma_bf16(lds16(ldsKt + off.tr[2 * sb] + db * 32 * 256), d0, acc[db]);
        acc[db] = mfma_bf16(lds16(ldsKt + off.tr[2 * sb + 1] + db * 32 * 256), d1, acc[db]);
      }
    }
  }
  store_acc_bf16<D>(make_rsrc((uint16_t*)a.out0 + j.base, a.slice_bytes), qrow, snb, acc, a.scale, g);
}

// dQ, fp32.

template <int D>
__global__ void __launch_bounds__(NT, 1) dq_f32_kernel(KArgs a) {
  __shared__ __attribute__((aligned(16))) char smem[2 * BLK * D * 4];
  char* ldsK = smem;
  char* ldsV = smem + BLK * D * 4;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i = lane & 31, g = lane >> 5;
  const Job j = decode_job(a);
  const uint32_t snb = (uint32_t)a.sn * 4;
  const rsrc_t rK = make_rsrc((const float*)a.k + j.base, a.slice_bytes);
  const rsrc_t rV = make_rsrc((const float*)a.v + j.base, a.slice_bytes);

  const int qrow = j.blk * BLK + 32 * w + i;
  f32x4 qf[D / 8], df[D / 8];
  load_frag_f32<D>(qf, make_rsrc((const float*)a.q + j.base, a.slice_bytes), qrow, snb, g);
  load_frag_f32<D>(df, make_rsrc((const float*)a.dout + j.base, a.slice_bytes), qrow, snb, g);
  float lse_t = 0.f, delta = 0.f;
  if (qrow < a.n) {
    lse_t = a.lse[stat_index(a, j, qrow)] * LOG2E;
    delta = a.delta[stat_index(a, j, qrow)];
  }
  F32Offsets<D> off;
  off.init(i, g);
  f32x16 acc[D / 32];
#pragma unroll
  for (int db = 0; db < D / 32; ++db) acc[db] = zero16();

  int t0, t1;
  tile_range(a, j.blk, t0, t1);
  for (int tt = t0; tt < t1; ++tt) {
    const int t = __builtin_amdgcn_readfirstlane(tt);
    const int kb = ((ci32_ptr)a.col)[t];
    __syncthreads();
    stage_rows_f32<D>(ldsK, rK, kb * BLK, snb, tid, true);
    stage_rows_f32<D>(ldsV, rV, kb * BLK, snb, tid, true);
    __syncthreads();
    const cu64_ptr mk = (cu64_ptr)a.lanes + ((int64_t)t * 4 + w) * 64;
#pragma unroll
    for (int sb = 0; sb < 4; ++sb) {
      SubMask m;
      m.load(mk, sb);
      f32x16 s = zero16(), dp = zero16();
#pragma unroll
      for (int u = 0; u < D / 8; ++u) {
        const f32x4 kx = *(const f32x4*)(ldsK + off.row[u & 3] + off.row_imm(sb, u));
        const f32x4 vx = *(const f32x4*)(ldsV + off.row[u & 3] + off.row_imm(sb, u));
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          s = mfma_f32(kx[e], qf[u][e], s);
          dp = mfma_f32(vx[e], df[u][e], dp);
        }
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float p = fast_exp2(fmaf(s[r], a.c2, -lse_t));
        p = select_lane(m.w[r], p, 0.f);
        dp[r] = p * (dp[r] - delta);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
#pragma unroll
        for (int db = 0; db < D / 32; ++db)
          acc[db] = mfma_f32(*(const float*)(ldsK + off.el[r & 3] + off.el_imm(sb, r, db)), dp[r], acc[db]);
      }
    }
  }
  store_acc_f32<D>(make_rsrc((float*)a.out0 + j.base, a.slice_bytes), qrow, snb, acc, a.scale, g);
}

// ------------------------------------------------------------------------------------------
// dK/dV, bf16: per key block over the transposed tile list; each workgroup owns its dK/dV rows,
// so there are no atomics (pallas_attn.py:187-215).

template <int D>
__global__ void __launch_bounds__(NT, 1) dkv_bf16_kernel(KArgs a) {
  __shared__ __attribute__((aligned(16))) char smem[4 * BLK * D * 2 + 2 * BLK * 4];
  char* ldsQ = smem;                     // [128][D] swizzled
  char* ldsQt = smem + BLK * D * 2;      // [D][128]
  char* ldsO = smem + 2 * BLK * D * 2;   // dO [128][D] swizzled
  char* ldsOt = smem + 3 * BLK * D * 2;  // dO^T [D][128]
  float* ldsL = (float*)(smem + 4 * BLK * D * 2);  // lse * log2(e) of the tile's 128 queries
  float* ldsDl = ldsL + BLK;                        // delta of the tile's queries
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i = lane & 31, g = lane >> 5;
  const Job j = decode_job(a);
  const uint32_t snb = (uint32_t)a.sn * 2;
  const rsrc_t rQ = make_rsrc((const uint16_t*)a.q + j.base, a.slice_bytes);
  const rsrc_t rO = make_rsrc((const uint16_t*)a.dout + j.base, a.slice_bytes);
  const float* lse = a.lse + stat_index(a, j, 0);
  const float* dl = a.delta + stat_index(a, j, 0);

  const int krow = j.blk * BLK + 32 * w + i;  // this lane's key
  u32x4 kf[D / 16], vf[D / 16];
  load_frag_bf16<D>(kf, make_rsrc((const uint16_t*)a.k + j.base, a.slice_bytes), krow, snb, g);
  load_frag_bf16<D>(vf, make_rsrc((const uint16_t*)a.v + j.base, a.slice_bytes), krow, snb, g);
  Bf16Offsets<D> off;
  off.init(i, g);
  f32x16 dk[D / 32], dv[D / 32];
#pragma unroll
  for (int db = 0; db < D / 32; ++db) {
    dk[db] = zero16();
    dv[db] = zero16();
  }

  int t0, t1;
  tile_range(a, j.blk, t0, t1);
  Bf16Stage<D> qs, os;
  const bool stager = Bf16Stage<D>::active(w);
  qs.init(w, lane, snb);
  os.init(w, lane, snb);
  float stat = 0.f;
  auto load_tile = [&](int t) {
    const int qb = ((ci32_ptr)a.col)[t];
    if (stager) {
      qs.load(rQ, qb * BLK, snb);
      os.load(rO, qb * BLK, snb);
    }
    const int row = qb * BLK + (tid & (BLK - 1));
    stat = 0.f;
    if (row < a.n) stat = tid < BLK ? lse[row] * LOG2E : dl[row];
  };
  if (t0 < t1) load_tile(t0);
  for (int tt = t0; tt < t1; ++tt) {
    const int t = __builtin_amdgcn_readfirstlane(tt);
    __syncthreads();
    if (stager) {
      qs.store_rows(ldsQ);
      qs.store_transposed(ldsQt);
      os.store_rows(ldsO);
      os.store_transposed(ldsOt);
    }
    (tid < BLK ? ldsL : ldsDl)[tid & (BLK - 1)] = stat;
    __syncthreads();
    if (t + 1 < t1) load_tile(t + 1);
    const cu64_ptr mk = (cu64_ptr)a.lanes + ((int64_t)t * 4 + w) * 64;
#pragma unroll
    for (int sb = 0; sb < 4; ++sb) {
      SubMask m;
      m.load(mk, sb);
      f32x16 s = zero16(), dp = zero16();
#pragma unroll
      for (int step = 0; step < D / 16; ++step) {
        s = mfma_bf16(lds16(ldsQ + off.row[step] + sb * 32 * (D * 2)), kf[step], s);
        dp = mfma_bf16(lds16(ldsO + off.row[step] + sb * 32 * (D * 2)), vf[step], dp);
      }
      // Statistics of the 16 queries in this lane's accumulator rows: 32*sb + 16*c + 8*g + 0..7.
      const int q0 = 32 * sb + 8 * g;
      float Lr[16], Dr[16];
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const f32x4 l0 = *(const f32x4*)(ldsL + q0 + 16 * c), l1 = *(const f32x4*)(ldsL + q0 + 16 * c + 4);
        const f32x4 d0 = *(const f32x4*)(ldsDl + q0 + 16 * c), d1 = *(const f32x4*)(ldsDl + q0 + 16 * c + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          Lr[8 * c + e] = l0[e];
          Lr[8 * c + 4 + e] = l1[e];
          Dr[8 * c + e] = d0[e];
          Dr[8 * c + 4 + e] = d1[e];
        }
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float p = fast_exp2(fmaf(s[r], a.c2, -Lr[r]));
        p = select_lane(m.w[r], p, 0.f);
        s[r] = p;
        dp[r] = p * (dp[r] - Dr[r]);
      }
      const bf16x8 p0 = pack_bf16(s, 0), p1 = pack_bf16(s, 1);
      const bf16x8 d0 = pack_bf16(dp, 0), d1 = pack_bf16(dp, 1);
#pragma unroll
      for (int db = 0; db < D / 32; ++db) {
        dv[db] = mfma_bf16(lds16(ldsOt + off.tr[2 * sb] + db * 32 * 256), p0, dv[db]);
        dv[db] = mfma_bf16(lds16(ldsOt + off.tr[2 * sb + 1] + db * 32 * 256), p1, dv[db]);
        dk[db] = mfma_bf16(lds16(ldsQt + off.tr[2 * sb] + db * 32 * 256), d0, dk[db]);
        dk[db] = mfma_bf16(lds16(ldsQt + off.tr[2 * sb + 1] + db * 32 * 256), d1, dk[db]);
      }
    }
  }
  store_acc_bf16<D>(make_rsrc((uint16_t*)a.out0 + j.base, a.slice_bytes), krow, snb, dk, a.scale, g);
  store_acc_bf16<D>(make_rsrc((uint16_t*)a.out1 + j.base, a.slice_bytes), krow, snb, dv, 1.f, g);
}

// dK/dV, fp32.

template <int D>
__global__ void __launch_bounds__(NT, 1) dkv_f32_kernel(KArgs a) {
  __shared__ __attribute__((aligned(16))) char smem[2 * BLK * D * 4 + 2 * BLK * 4];
  char* ldsQ = smem;                // [128][D] swizzled
  char* ldsO = smem + BLK * D * 4;  // dO [128][D] swizzled
  float* ldsL = (float*)(smem + 2 * BLK * D * 4);
  float* ldsDl = ldsL + BLK;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i = lane & 31, g = lane >> 5;
  const Job j = decode_job(a);
  const uint32_t snb = (uint32_t)a.sn * 4;
  const rsrc_t rQ = make_rsrc((const float*)a.q + j.base, a.slice_bytes);
  const rsrc_t rO = make_rsrc((const float*)a.dout + j.base, a.slice_bytes);
  const float* lse = a.lse + stat_index(a, j, 0);
  const float* dl = a.delta + stat_index(a, j, 0);

  const int krow = j.blk * BLK + 32 * w + i;
  f32x4 kf[D / 8], vf[D / 8];
  load_frag_f32<D>(kf, make_rsrc((const float*)a.k + j.base, a.slice_bytes), krow, snb, g);
  load_frag_f32<D>(vf, make_rsrc((const float*)a.v + j.base, a.slice_bytes), krow, snb, g);
  F32Offsets<D> off;
  off.init(i, g);
  f32x16 dk[D / 32], dv[D / 32];
#pragma unroll
  for (int db = 0; db < D / 32; ++db) {
    dk[db] = zero16();
    dv[db] = zero16();
  }

  int t0, t1;
  tile_range(a, j.blk, t0, t1);
  for (int tt = t0; tt < t1; ++tt) {
    const int t = __builtin_amdgcn_readfirstlane(tt);
    const int qb = ((ci32_ptr)a.col)[t];
    __syncthreads();
    stage_rows_f32<D>(ldsQ, rQ, qb * BLK, snb, tid, true);
    stage_rows_f32<D>(ldsO, rO, qb * BLK, snb, tid, true);
    {
      const int row = qb * BLK + (tid & (BLK - 1));
      float stat = 0.f;
      if (row < a.n) stat = tid < BLK ? lse[row] * LOG2E : dl[row];
      (tid < BLK ? ldsL : ldsDl)[tid & (BLK - 1)] = stat;
    }
    __syncthreads();
    const cu64_ptr mk = (cu64_ptr)a.lanes + ((int64_t)t * 4 + w) * 64;
#pragma unroll
    for (int sb = 0; sb < 4; ++sb) {
      SubMask m;
      m.load(mk, sb);
      f32x16 s = zero16(), dp = zero16();
#pragma unroll
      for (int u = 0; u < D / 8; ++u) {
        const f32x4 qx = *(const f32x4*)(ldsQ + off.row[u & 3] + off.row_imm(sb, u));
        const f32x4 ox = *(const f32x4*)(ldsO + off.row[u & 3] + off.row_imm(sb, u));
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          s = mfma_f32(qx[e], kf[u][e], s);
          dp = mfma_f32(ox[e], vf[u][e], dp);
        }
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int qq = element_col(sb, r, g);
        float p = fast_exp2(fmaf(s[r], a.c2, -ldsL[qq]));
        p = select_lane(m.w[r], p, 0.f);
        s[r] = p;
        dp[r] = p * (dp[r] - ldsDl[qq]);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
#pragma unroll
        for (int db = 0; db < D / 32; ++db) {
          dv[db] = mfma_f32(*(const float*)(ldsO + off.el[r & 3] + off.el_imm(sb, r, db)), s[r], dv[db]);
          dk[db] = mfma_f32(*(const float*)(ldsQ + off.el[r & 3] + off.el_imm(sb, r, db)), dp[r], dk[db]);
        }
      }
    }
  }
  store_acc_f32<D>(make_rsrc((float*)a.out0 + j.base, a.slice_bytes), krow, snb, dk, a.scale, g);
  store_acc_f32<D>(make_rsrc((float*)a.out1 + j.base, a.slice_bytes), krow, snb, dv, 1.f, g);
}

// ------------------------------------------------------------------------------------------
// delta = rowsum(o * dout) (pallas_attn.py:278): L lanes per (batch, head, row), 16 B per lane.

template <typename T, int D>
__global__ void __launch_bounds__(NT) delta_kernel(KArgs a) {
  constexpr int EPC = 16 / (int)sizeof(T);
  constexpr int L = D / EPC;
  const int64_t gid = (int64_t)blockIdx.x * NT + threadIdx.x;
  const int64_t item = gid / L;
  const int part = (int)(gid % L);
  const int64_t total = (int64_t)a.batch * a.heads * a.n;
  float sum = 0.f;
  if (item < total) {
    const int row = (int)(item % a.n);
    const int64_t bh = item / a.n;
    const int h = (int)(bh % a.heads), b = (int)(bh / a.heads);
    const int64_t off = (int64_t)b * a.sb + (int64_t)h * a.sh + (int64_t)row * a.sn + part * EPC;
    const u32x4 x = *(const u32x4*)((const T*)a.o + off);
    const u32x4 y = *(const u32x4*)((const T*)a.dout + off);
    if constexpr (sizeof(T) == 4) {
      const f32x4 fx = __builtin_bit_cast(f32x4, x), fy = __builtin_bit_cast(f32x4, y);
#pragma unroll
      for (int e = 0; e < 4; ++e) sum += fx[e] * fy[e];
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        sum += __uint_as_float(x[e] << 16) * __uint_as_float(y[e] << 16);
        sum += __uint_as_float(x[e] & 0xffff0000u) * __uint_as_float(y[e] & 0xffff0000u);
      }
    }
  }
#pragma unroll
  for (int o = L / 2; o > 0; o >>= 1) sum += __shfl_xor(sum, o);
  if (item < total && part == 0) a.lse_out[item] = sum;
}

template <int D>
hipError_t launch_d(Kind kind, int dtype, const KArgs& a, hipStream_t stream) {
  const dim3 block(NT);
  if (kind == Kind::kDelta) {
    const int64_t lanes = (int64_t)a.batch * a.heads * a.n * (dtype ? D / 8 : D / 4);
    const dim3 dgrid((unsigned)((lanes + NT - 1) / NT));
    if (dtype) hipLaunchKernelGGL((delta_kernel<uint16_t, D>), dgrid, block, 0, stream, a);
    else hipLaunchKernelGGL((delta_kernel<float, D>), dgrid, block, 0, stream, a);
    return hipGetLastError();
  }
  const dim3 grid((unsigned)a.n_blocks * (unsigned)(a.batch * a.heads));
  switch (kind) {
    case Kind::kFwd:
      if (dtype) hipLaunchKernelGGL(fwd_bf16_kernel<D>, grid, block, 0, stream, a);
      else hipLaunchKernelGGL(fwd_f32_kernel<D>, grid, block, 0, stream, a);
      break;
    case Kind::kDq:
      if (dtype) hipLaunchKernelGGL(dq_bf16_kernel<D>, grid, block, 0, stream, a);
      else hipLaunchKernelGGL(dq_f32_kernel<D>, grid, block, 0, stream, a);
      break;
    case Kind::kDkv:
      if (dtype) hipLaunchKernelGGL(dkv_bf16_kernel<D>, grid, block, 0, stream, a);
      else hipLaunchKernelGGL(dkv_f32_kernel<D>, grid, block, 0, stream, a);
      break;
    default:
      break;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch(Kind kind, int dtype, int head_dim, const KArgs& a, hipStream_t stream) {
  switch (head_dim) {
    case 32: return launch_d<32>(kind, dtype, a, stream);
    case 64: return launch_d<64>(kind, dtype, a, stream);
    case 128: return launch_d<128>(kind, dtype, a, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace fwn
