// Device-side building blocks shared by the bf16 and fp32 attention kernels (gfx950 only).
//
// Conventions used by every kernel:
//   - One workgroup = 4 waves = one 128-row block of queries (forward, dQ) or keys (dK/dV) for one
//     (batch, head); wave w owns rows 32w..32w+31 of the block; lane l has i = l % 32, g = l / 32.
//   - The first contraction is computed transposed, X^T[col][row] (S^T = K Q^T in the forward),
//     so the 32x32 MFMA accumulator column (lane % 32) is the wave's own row and softmax
//     statistics are per lane. Its A-operand rows are loaded in the order sigma(i), which makes
//     accumulator register r of lane group g hold column element_col(sb, r, g): 8 consecutive
//     columns per lane group and 16-column chunk, i.e. the B-operand layout of the second
//     contraction. P and dS therefore go from accumulator to MFMA operand in registers.
//   - Global memory is read through raw buffer resources, one per (batch, head) slice; the
//     hardware range check returns zeros for rows >= n and drops their stores.
//   - Tile masks are one 64-bit word per lane and wave (fwn_tiles_prepare): bit e says whether
//     accumulator element e (sub-block e / 16, register e % 16) of this lane is a valid key. A
//     wave fetches its 512 bytes per tile with one coalesced vector load, issued a tile ahead;
//     a valid element is kept with a sign-extracted bit and one AND or bitfield insert.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "attn_kernels.h"

namespace fwn {
namespace dev {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __amdgpu_buffer_rsrc_t rsrc_t;

typedef const __attribute__((address_space(4))) uint64_t* cu64_ptr;
typedef const __attribute__((address_space(4))) uint32_t* cu32_ptr;
typedef const __attribute__((address_space(4))) int32_t* ci32_ptr;
typedef __attribute__((address_space(3))) char lds_char;

constexpr int BLK = 128;
constexpr int NT = 256;
constexpr int RSRC_DW3 = 0x00020000;  // raw buffer, 32-bit dword format (gfx9 family)
constexpr float LOG2E = 1.4426950408889634f;
constexpr float LN2 = 0.6931471805599453f;

// Operand row that MFMA row i of a 32-row sub-block loads.
__device__ __forceinline__ int sigma(int i) {
  return ((i >> 4) << 4) | (((i >> 2) & 1) << 3) | (((i >> 3) & 1) << 2) | (i & 3);
}

// Column (key or query) within a 128-wide tile held by accumulator register r of sub-block sb.
__device__ __forceinline__ int element_col(int sb, int r, int g) { return 32 * sb + 16 * (r >> 3) + 8 * g + (r & 7); }

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


// Waits for every outstanding vector-memory operation (s_waitcnt vmcnt(0); expcnt and lgkmcnt
// left free).
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// 2^x on the hardware transcendental unit (V_EXP_F32); callers fold log2(e) into their scales.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Workgroup barrier for hand-overs through LDS: an LDS-scoped release/acquire around s_barrier.
// __syncthreads() waits for every outstanding global load as well; this one waits for the
// wave's LDS operations, plus any global load that writes LDS (a tile copy still in flight)
// where the compiler sees one outstanding. A barrier that never waits for copies (inline
// s_waitcnt lgkmcnt(0); s_barrier) measured 2% slower in an earlier dK/dV kernel.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

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

struct Job {
  int blk;
  int b, h, bh;
  int t0, t1;    // tile range of this work item, clamped to [0, n_tiles)
  int part;      // partial slot, or -1 when the item covers its whole block
  int64_t base;   // element offset of (b, h) in q, k, v, dq, dk, dv
  int64_t obase;  // element offset of (b, h) in o, dout
  bool skip;     // an empty entry of the order table: the workgroup does nothing
};

// Without an order table, workgroups are dealt round-robin over the 8 XCDs, each with its own
// L2. Jobs are ordered (batch, head) major, then work items in block order, and XCD x gets a
// contiguous range of them, so the workgroups resident on one XCD work on neighbouring blocks of
// one head and share their K/V tiles in that XCD's L2. The map from workgroup id to job is a
// bijection for any count.
//
// With an order table (fwn_tiles_order_fill), workgroup `pid` runs the (batch * heads + head,
// item) pair of entry pid; the host has placed each XCD's jobs at the ids pid = x mod 8 it
// serves. Entries outside the call's pairs or items are skipped, so a malformed table cannot
// send a workgroup outside the tensors.
__device__ __forceinline__ Job decode_job(const KArgs& a, int pid = -1) {
  Job j;
  if (pid < 0) pid = blockIdx.x;
  int slot;
  if (a.order) {
    j.bh = ((ci32_ptr)a.order)[2 * pid];
    slot = ((ci32_ptr)a.order)[2 * pid + 1];
    j.skip = (unsigned)j.bh >= (unsigned)(a.batch * a.heads) || (unsigned)slot >= (unsigned)a.n_items;
    if (j.skip) {
      j.bh = 0;
      slot = 0;
    }
  } else {
    const int total = a.n_items * a.batch * a.heads;
    const int xcd = pid & 7, local = pid >> 3;
    const int small = total >> 3, rem = total & 7;
    const int job = xcd < rem ? xcd * (small + 1) + local : rem * (small + 1) + (xcd - rem) * small + local;
    j.bh = job / a.n_items;
    slot = job - j.bh * a.n_items;
    j.skip = false;
  }
  const ci32_ptr item = (ci32_ptr)a.items + 4 * slot;
  j.blk = item[0];
  j.t0 = item[1] < 0 ? 0 : item[1];
  j.t1 = item[2] > a.n_tiles ? a.n_tiles : item[2];
  j.part = item[3];
  // A malformed item cannot write outside the outputs or the workspace: an out-of-range block
  // gets no tiles (its rows are >= n, so the range-checked stores drop), an out-of-range slot
  // writes the outputs directly.
  if ((unsigned)j.blk >= (unsigned)a.n_blocks) j.t1 = j.t0;
  if (j.part >= a.n_parts) j.part = -1;
  j.b = j.bh / a.heads;
  j.h = j.bh - j.b * a.heads;
  j.base = (int64_t)j.b * a.sb + (int64_t)j.h * a.sh;
  j.obase = (int64_t)j.b * a.osb + (int64_t)j.h * a.osh;
  return j;
}

__device__ __forceinline__ void tile_range(const KArgs&, const Job& j, int& t0, int& t1) {
  t0 = j.t0;
  t1 = j.t1;
}

// Buffer resource of this item's partial slot for its (batch, head): [128][D] float32 rows
// (O, dQ or dK), then [128][D] (dV) or the forward's row max [128] and row sum [128].
template <int D>
__device__ __forceinline__ rsrc_t part_slot(const KArgs& a, const Job& j) {
  constexpr int64_t words = 128 * (2 * D + 2);
  return make_rsrc(a.work + ((int64_t)j.part * a.batch * a.heads + j.bh) * words, (uint32_t)(words * 4));
}

__device__ __forceinline__ void store_f32(rsrc_t r, uint32_t byte_off, float x) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, x), r, (int)byte_off, 0, 0);
}


__device__ __forceinline__ int64_t stat_index(const KArgs& a, const Job& j, int row) {
  return ((int64_t)j.b * a.heads + j.h) * a.n + row;
}

// This lane's validity bits for tile t (wave w): bit e = element e. Fully valid tiles hold
// all-ones words, so masks are applied unconditionally (no branch).
__device__ __forceinline__ u32x2 tile_bits(const KArgs& a, int t, int w, int lane) {
  return *(const u32x2*)(a.lanes + ((int64_t)t * 4 + w) * 64 + lane);
}

// All ones if element (sb, r) is valid for this lane, else 0: one v_bfe_i32 of one bit.
__device__ __forceinline__ uint32_t elem_keep(const u32x2& bits, int sb, int r) {
  const int e = 16 * sb + r;
  return __builtin_amdgcn_sbfe(bits[e >> 5], (uint32_t)(e & 31), 1u);
}

// The tile's 16 group bits: bit 4r + c is set when rows 32r..32r+31 have a valid element in
// columns 32c..32c+31. A wave owning row group r computes only the column groups in
// (bits >> 4r) & 15; the others would add p = 0.
// Read through the constant address space, so a uniform index becomes a scalar load and the
// value an SGPR (the kernels branch on it).
__device__ __forceinline__ uint32_t tile_groups(const KArgs& a, int t) {
  return ((const __attribute__((address_space(4))) uint32_t*)a.groups)[t];
}

// The tile's 32 half bits: bit 8r + 2c + h is set when rows 32r..32r+31 have a valid element in
// columns 32c + 16h .. +15. Accumulator registers 8h..8h+7 of sub-block c hold exactly those 16
// columns (element_col), so a clear bit skips their dS work and the dQ MFMAs they feed; they
// would add exact zeros. Lists prepared without halves read all ones.
__device__ __forceinline__ uint32_t tile_halves(const KArgs& a, int t) {
  return a.halves ? ((const __attribute__((address_space(4))) uint32_t*)a.halves)[t] : ~0u;
}

// Masks of the 16-key dK/dV kernel, whose lane l holds key l % 16 of its wave's 16 and queries
// 4g + r, 16 + 4g + r (g = l / 16, r < 4) of a 32-query group. This lane's mask word of tile 0 for
// 16-key group kg (add 256 words per tile): the word of 32-row wave kg / 2, lane
// 32 (g / 2) + 16 (kg % 2) + l % 16, which, shifted right by 4 (g % 2), holds element (query
// group c, half m, r) at bit 16c + 8m + r.
__device__ __forceinline__ const uint64_t* key_mask_words(const KArgs& a, int kg, int g, int t16) {
  return a.lanes + (int64_t)(kg >> 1) * 64 + 32 * (g >> 1) + 16 * (kg & 1) + t16;
}

// Column groups with a valid element in any row group.
__device__ __forceinline__ uint32_t any_rows(uint32_t g) { return (g | g >> 4 | g >> 8 | g >> 12) & 15u; }

// x where kept, -inf elsewhere (one v_bitop3_b32).
__device__ __forceinline__ float keep_or_ninf(float x, uint32_t keep) {
  return __builtin_bit_cast(float, (__builtin_bit_cast(uint32_t, x) & keep) | (0xff800000u & ~keep));
}

// x where kept, +0 elsewhere (one v_and_b32). The empty asm hides that `keep` is a sign-extended
// bit; otherwise the compiler turns the AND into a bit test, a compare and a v_cndmask (three
// instructions and a VCC hazard instead of one).
__device__ __forceinline__ float keep_or_zero(float x, uint32_t keep) {
  asm("" : "+v"(keep));
  return __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, x) & keep);
}

// Online softmax of the forward kernels (pallas_attn.py:125-131) with a lazily moved reference
// max. s[sb][r] holds this lane's masked logits (raw q.k, -inf where masked); on return it holds
// p = exp2(s*c2 - m) for the lane's reference max m. m moves only when some lane of the wave sees
// a logit more than kLazyMax above its m (a wave-uniform decision); otherwise p <= 2^kLazyMax,
// the accumulators keep their scale and the caller skips the rescale. O and l always share m, so
// O / l and lse = m + log2 l are unchanged up to rounding. Returns true when m moved; `corr` is
// then the factor the caller applies to its accumulators (l is rescaled here).
constexpr float kLazyMax = 8.f;

struct SoftmaxState {
  float m;  // reference max of s*c2 (log2 domain), -inf before the first valid key
  float l;  // running sum of exp2(s*c2 - m) over this lane's half of the keys
};

// The lazy move itself, from this lane's max over its half of the row's logits. Lanes i and
// i + 32 hold one row and share m, and x * c2 is monotonic, so "some lane's half-row max exceeds
// m + kLazyMax" is exactly "some row's max does": the wave-uniform decision needs no cross-lane
// step, and the row max (one lane exchange) is formed only when m moves.
__device__ __forceinline__ bool lazy_move(float mx_half, SoftmaxState& st, float c2, float& corr) {
  corr = 1.f;
  if (__builtin_amdgcn_ballot_w64(mx_half * c2 > st.m + kLazyMax) == 0) return false;
  const float mxs = fmaxf(mx_half, __shfl_xor(mx_half, 32)) * c2;
  const float m_new = fmaxf(st.m, mxs);
  corr = fast_exp2(st.m - (m_new == -__builtin_inff() ? 0.f : m_new));
  st.l *= corr;
  st.m = m_new;
  return true;
}

// The first NSB entries of s take part (all of them by default).
template <int NSB = -1, int CAP>
__device__ __forceinline__ bool softmax_tile(f32x16 (&s)[CAP], SoftmaxState& st, float c2, float& corr) {
  constexpr int N = NSB < 0 ? CAP : NSB;
  static_assert(N >= 1 && N <= CAP, "sub-block count");
  const float ninf = -__builtin_inff();
  float mx = s[0][0];
#pragma unroll
  for (int sb = 0; sb < N; ++sb)
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[sb][r]);
  const bool moved = lazy_move(mx, st, c2, corr);
  const float base = st.m == ninf ? 0.f : st.m;
  float sum = 0.f;
#pragma unroll
  for (int sb = 0; sb < N; ++sb)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float p = fast_exp2(fmaf(s[sb][r], c2, -base));
      s[sb][r] = p;
      sum += p;
    }
  st.l += sum;
  return moved;
}

// First half of softmax_live: the row max over the sub-blocks in `live`, the lazy move of the
// reference max and the rescale of l. Returns whether m moved (`corr` rescales the caller's
// accumulators); the caller then computes p = exp2(s * c2 - base) per sub-block with
// base = softmax_base(st) and adds the row sums to st.l itself.
__device__ __forceinline__ bool softmax_rebase(const f32x16 (&s)[4], uint32_t live, SoftmaxState& st, float c2,
                                               float& corr) {
  const float ninf = -__builtin_inff();
  float mx = ninf;
#pragma unroll
  for (int sb = 0; sb < 4; ++sb)
    if (live >> sb & 1u) {
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[sb][r]);
    }
  const bool moved = lazy_move(mx, st, c2, corr);
  return moved;
}

__device__ __forceinline__ float softmax_base(const SoftmaxState& st) {
  return st.m == -__builtin_inff() ? 0.f : st.m;
}

// softmax_tile over the sub-blocks in `live` only (a nonzero wave-uniform set); the others are
// neither read nor written.
template <int N>
__device__ __forceinline__ bool softmax_live(f32x16 (&s)[N], uint32_t live, SoftmaxState& st, float c2,
                                             float& corr) {
  const float ninf = -__builtin_inff();
  float mx = ninf;
#pragma unroll
  for (int sb = 0; sb < N; ++sb)
    if (live >> sb & 1u) {
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[sb][r]);
    }
  const bool moved = lazy_move(mx, st, c2, corr);
  const float base = st.m == ninf ? 0.f : st.m;
  float sum = 0.f;
#pragma unroll
  for (int sb = 0; sb < N; ++sb)
    if (live >> sb & 1u) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = fast_exp2(fmaf(s[sb][r], c2, -base));
        s[sb][r] = p;
        sum += p;
      }
    }
  st.l += sum;
  return moved;
}

// Natural log-sum-exp of the scaled logits: (m + log2 l) * ln 2 (pallas_attn.py:140-141).
__device__ __forceinline__ void write_lse(const KArgs& a, const Job& j, int row, const SoftmaxState& st, float ltot) {
  if (a.lse_out && row < a.n) {
    const float lse = (st.m + __builtin_amdgcn_logf(fmaxf(ltot, 1e-30f))) * LN2;
    a.lse_out[stat_index(a, j, row)] = lse;
  }
}

// Stores a transposed accumulator (rows d, column = this lane's row) as bf16, times `mul`. The
// NB accumulators hold the 32-column blocks db0 .. db0 + NB - 1.
template <int D, int NB = D / 32>
__device__ __forceinline__ void store_acc_bf16(rsrc_t r, int row, uint32_t snb, const f32x16 (&acc)[NB],
                                               float mul, int g, int db0 = 0) {
#pragma unroll
  for (int db = 0; db < NB; ++db) {
#pragma unroll
    for (int k4 = 0; k4 < 4; ++k4) {
      const int d = 32 * (db0 + db) + 8 * k4 + 4 * g;
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

// Stores a transposed accumulator as float32, times `mul` (blocks db0 .. db0 + NB - 1).
template <int D, int NB = D / 32>
__device__ __forceinline__ void store_acc_f32(rsrc_t r, int row, uint32_t snb, const f32x16 (&acc)[NB], float mul,
                                              int g, int db0 = 0) {
#pragma unroll
  for (int db = 0; db < NB; ++db) {
#pragma unroll
    for (int k4 = 0; k4 < 4; ++k4) {
      const int d = 32 * (db0 + db) + 8 * k4 + 4 * g;
      f32x4 w;
#pragma unroll
      for (int e = 0; e < 4; ++e) w[e] = acc[db][4 * k4 + e] * mul;
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, w), r,
                                             (int)((uint32_t)row * snb + (uint32_t)(4 * d)), 0, 0);
    }
  }
}

// Forward partial epilogue: unnormalised O^T rows, the row max (log2 domain) and the row sum.
// `row` is the row within the block.
template <int D>
__device__ __forceinline__ void store_fwd_partial(const KArgs& a, const Job& j, int row, const f32x16 (&o)[D / 32],
                                                  float m, float ltot, int g) {
  const rsrc_t r = part_slot<D>(a, j);
  store_acc_f32<D>(r, row, D * 4, o, 1.f, g);
  if (g == 0) {
    store_f32(r, (uint32_t)(128 * D + row) * 4, m);
    store_f32(r, (uint32_t)(128 * D + 128 + row) * 4, ltot);
  }
}

// Backward partial epilogue: unscaled accumulator rows into the first (which = 0: dQ, dK) or
// second (which = 1: dV) half of the slot.
template <int D, int NB = D / 32>
__device__ __forceinline__ void store_bwd_partial(const KArgs& a, const Job& j, int row, const f32x16 (&acc)[NB],
                                                  int which, int g, int db0 = 0) {
  store_acc_f32<D, NB>(part_slot<D>(a, j), row + 128 * which, D * 4, acc, 1.f, g, db0);
}

}  // namespace dev
}  // namespace fwn
