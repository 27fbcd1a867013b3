// float32 attention kernels for gfx950: forward, dQ, dK/dV (V_MFMA_F32_32X32X2_F32, and
// V_MFMA_F32_16X16X4F32 for the 16-key dK/dV at head_dim 128; full fp32 products and
// accumulation), and the delta pre-pass for both dtypes.
//
// fp32 MFMA operands are one element per lane, so the second contraction's A operand (V^T, K^T,
// Q^T, dO^T) is read element-wise straight from the row-major LDS tile; no transposed copy is
// needed. Tiles stream into LDS by LDS DMA, double-buffered: in 64-row halves for the backward
// kernels (HalfDma), in 32-row key groups for the forward (GroupDma).
//
// Reference: pallas_attn.py:112-141 (forward), 161-215 (dQ, dK/dV), 274-311 (VJP driver).
#include "attn_device.h"

namespace fwn {
namespace {

using namespace dev;

// 3-bit variant for fp32 tiles: keeps 32-column blocks of a row inside one aligned 128 bytes.
__device__ __forceinline__ int swz_row3(int row) { return (row & 3) | (((row >> 3) & 1) << 2); }

// ------------------------------------------------------------------------------------------
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

// Schedules a loop of N steps, each with R LDS reads followed by the M MFMAs that consume them,
// so that the reads run two steps ahead of their MFMAs: with one wave per SIMD nothing else fills
// the MFMA pipe while a wave waits for a read it issued just before use. (The compiler, left to
// itself, issues each step's reads right before its MFMAs.) Place after the reads and MFMAs it
// orders, in the same basic block.
template <int N, int R, int M>
__device__ __forceinline__ void sched_reads_ahead() {
  __builtin_amdgcn_sched_group_barrier(0x100, 2 * R, 0);  // the reads of steps 0 and 1
#pragma unroll
  for (int k = 0; k < N - 2; ++k) {
    __builtin_amdgcn_sched_group_barrier(0x008, M, 0);  // step k's MFMAs
    __builtin_amdgcn_sched_group_barrier(0x100, R, 0);  // step k + 2's reads
  }
  __builtin_amdgcn_sched_group_barrier(0x008, 2 * M, 0);  // the last two steps' MFMAs
}

// Copies rows 64h .. 64h + 63 of a 128-row fp32 tile (rows of 4D bytes, 16-byte chunks swizzled
// by swz_row3, or plain) from global rows row0 + 64h .. into a 64-row half buffer with the buffer
// unit's LDS DMA, so the copy needs no registers and runs while the other half is computed. Only
// the 32-row groups in `live` (tile group bits 2h and 2h + 1) are copied. Wave w of 4 issues the
// 1 KB instructions k = w + 4m; instruction k fills half rows kR .. kR + R - 1 (R = 1024 / 4D),
// which lie in one group, and lane l the chunk that belongs at its position. The lane's part of
// the global offset depends only on the parity of m (the swizzle's row bit 3 at D = 128), so two
// registers hold it; the per-instruction offsets are formed at the copy and not hoisted out of
// the tile loop, where they would hold 2 registers per instruction.
template <int D>
struct HalfDma {
  static constexpr int R = 1024 / (D * 4);
  static constexpr int CPR = D / 4;
  static constexpr int NI = 64 / R;
  uint32_t lo[2];

  __device__ __forceinline__ void init(int w, int lane, uint32_t snb, bool swizzle) {
    const int rl = lane / CPR, pc = lane % CPR;
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const int row = (w + 4 * m) * R + rl;  // same low bits for every h and every m of this parity
      lo[m] = (uint32_t)rl * snb + (uint32_t)((swizzle ? pc ^ swz_row3(row) : pc) << 4);
    }
  }

  __device__ __forceinline__ void issue(rsrc_t r, char* half, int row0, uint32_t snb, int w, int h,
                                        uint32_t live) const {
    uint32_t base = (uint32_t)(uintptr_t)half;
    asm volatile("" : "+s"(base));
    uint32_t l0 = lo[0], l1 = lo[1];
    asm volatile("" : "+v"(l0), "+v"(l1));
#pragma unroll
    for (int m = 0; m < NI / 4; ++m) {
      const int k = w + 4 * m;
      if (!(live >> (2 * h + ((k * R) >> 5)) & 1u)) continue;
      const uint32_t src = (uint32_t)(row0 + 64 * h + k * R) * snb + ((m & 1) ? l1 : l0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)(uintptr_t)(base + 1024u * k),
                                               16, (int)src, 0, 0, 0);
    }
  }
};

// ------------------------------------------------------------------------------------------
// Copies one 32-row key group of a 128-row fp32 tile (global rows row0 ..) into a 32-row group
// buffer with the buffer unit's LDS DMA, in the layout of HalfDma's rows 0-31 (the swizzle
// depends on the row modulo 16). Wave w of 4 issues instructions k = w + 4m, each filling rows
// kR .. kR + R - 1; the lane's part of the source offset depends on the parity of m only.
template <int D>
struct GroupDma {
  static constexpr int R = 1024 / (D * 4);
  static constexpr int CPR = D / 4;
  static constexpr int NI = 32 / R;
  uint32_t lo[2];

  __device__ __forceinline__ void init(int w, int lane, uint32_t snb, bool swizzle) {
    const int rl = lane / CPR, pc = lane % CPR;
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const int row = (w + 4 * m) * R + rl;
      lo[m] = (uint32_t)rl * snb + (uint32_t)((swizzle ? pc ^ swz_row3(row) : pc) << 4);
    }
  }

  __device__ __forceinline__ void issue(rsrc_t r, char* buf, int row0, uint32_t snb, int w) const {
    uint32_t base = (uint32_t)(uintptr_t)buf;
    asm volatile("" : "+s"(base));
    uint32_t l0 = lo[0], l1 = lo[1];
    asm volatile("" : "+v"(l0), "+v"(l1));
#pragma unroll
    for (int m = 0; m < NI / 4; ++m) {
      const int k = w + 4 * m;
      const uint32_t src = (uint32_t)(row0 + k * R) * snb + ((m & 1) ? l1 : l0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)(uintptr_t)(base + 1024u * k),
                                               16, (int)src, 0, 0, 0);
    }
  }
};

// Forward, fp32, two workgroups per CU, streamed by 32-key group: the work item's steps are its
// (tile, key group) pairs in which some wave has a valid element; each step's K and V rows (32 KB
// at D = 128) go into one of two group buffers, the copy of step s + 1 running while step s is
// computed, one barrier per step. Groups no wave needs cost neither a copy nor a barrier.
template <int D>
__global__ void __launch_bounds__(NT, 2) fwd_f32g_kernel(KArgs a) {
  constexpr int GB = 32 * D * 4;  // bytes of 32 rows of K or V
  __shared__ __attribute__((aligned(1024))) char gb0[2 * GB];  // K group (swizzled) | V group (plain)
  __shared__ __attribute__((aligned(1024))) char gb1[2 * GB];
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i = lane & 31, g = lane >> 5;
  const Job j = decode_job(a);
  if (j.skip) return;  // an empty entry of the order table
  const uint32_t snb = (uint32_t)a.sn * 4;
  const rsrc_t rK = make_rsrc((const float*)a.k + j.base, a.slice_bytes);
  const rsrc_t rV = make_rsrc((const float*)a.v + j.base, a.slice_bytes);
  const int qrow = j.blk * BLK + 32 * w + i;
  f32x4 qf[D / 8];
  load_frag_f32<D>(qf, make_rsrc((const float*)a.q + j.base, a.slice_bytes), qrow, snb, g);
  F32Offsets<D> off;
  off.init(i, g);
  GroupDma<D> dmaK, dmaV;
  dmaK.init(w, lane, snb, true);
  dmaV.init(w, lane, snb, false);
  f32x16 o[D / 32];
#pragma unroll
  for (int db = 0; db < D / 32; ++db) o[db] = zero16();
  SoftmaxState st{-__builtin_inff(), 0.f};

  // Key group sb of a tile from group buffer gb. hv: the group's 16-key halves with a valid
  // element for this wave (bit h: keys 16 h .. 16 h + 15, registers 8 h .. 8 h + 7 of S); a clear
  // half has p = 0 throughout and skips its PV MFMAs.
  auto group = [&](int sb, const char* gb, u32x2 mb, uint32_t hv) {
    const char* ldsK = gb;
    const char* ldsV = gb + GB;
    f32x16 s[1];
    s[0] = zero16();
#pragma unroll
    for (int u = 0; u < D / 8; ++u) {
      const f32x4 kx = *(const f32x4*)(ldsK + off.row[u & 3] + off.row_imm(0, u));
#pragma unroll
      for (int e = 0; e < 4; ++e) s[0] = mfma_f32(kx[e], qf[u][e], s[0]);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) s[0][r] = keep_or_ninf(s[0][r], elem_keep(mb, sb, r));
    float corr;
    if (softmax_live<1>(s, 1u, st, a.c2, corr)) {
#pragma unroll
      for (int db = 0; db < D / 32; ++db) o[db] *= corr;
    }
#pragma unroll
    for (int h = 0; h < 2; ++h)
      if (hv >> h & 1u) {
#pragma unroll
        for (int r = 8 * h; r < 8 * h + 8; ++r) {
#pragma unroll
          for (int db = 0; db < D / 32; ++db)
            o[db] = mfma_f32(*(const float*)(ldsV + off.el_plain + off.el_imm(0, r, db)), s[0][r], o[db]);
        }
      }
  };

  int t0, t1;
  tile_range(a, j, t0, t1);
  // Step iterator: tile ti, its key groups not taken yet in rem (wave-uniform scalars).
  int ti = t0 - 1;
  uint32_t rem = 0u;
  auto take = [&](int& t, int& c) -> bool {
    while (rem == 0u) {
      if (++ti >= t1) return false;
      rem = any_rows(tile_groups(a, ti));
    }
    t = ti;
    c = __builtin_ctz(rem);
    rem &= rem - 1u;
    return true;
  };
  auto copy = [&](char* gb, int t, int c) {
    const int row0 = ((ci32_ptr)a.col)[t] * BLK + 32 * c;
    dmaK.issue(rK, gb, row0, snb, w);
    dmaV.issue(rV, gb + GB, row0, snb, w);
  };
  int tc = 0, cc = 0, tn = 0, cn = 0;
  bool vc = take(tc, cc), vn = false;
  u32x2 mbc = {0u, 0u}, mbn = {0u, 0u};
  if (vc) {
    copy(gb0, tc, cc);
    mbc = tile_bits(a, tc, w, lane);
    vn = take(tn, cn);
  }
  // One step: step (tc, cc) is in `cur`; the copy of step (tn, cn) goes into `nxt`.
  auto step = [&](char* cur, char* nxt) {
    wait_vmem();      // this wave's part of the current step (and its mask bits)
    __syncthreads();  // the step landed; every wave is done with the previous step's buffer
    if (vn) {
      copy(nxt, tn, cn);
      mbn = tn != tc ? tile_bits(a, tn, w, lane) : mbc;
    }
    const uint32_t live = tile_groups(a, tc) >> (4 * w) & 15u;
    if (live >> cc & 1u) group(cc, cur, mbc, tile_halves(a, tc) >> (8 * w + 2 * cc) & 3u);
    tc = tn;
    cc = cn;
    mbc = mbn;
    vc = vn;
    vn = vc && take(tn, cn);
  };
  while (vc) {
    step(gb0, gb1);
    if (!vc) break;
    step(gb1, gb0);
  }
  const float ltot = st.l + __shfl_xor(st.l, 32);
  if (j.part >= 0) {
    store_fwd_partial<D>(a, j, 32 * w + i, o, st.m, ltot, g);
    return;
  }
  const float inv = ltot > 0.f ? 1.f / ltot : 0.f;
  store_acc_f32<D>(make_rsrc((float*)a.out0 + j.obase, a.oslice_bytes), qrow, (uint32_t)a.osn * 4, o, inv, g);
  if (g == 0) write_lse(a, j, qrow, st, ltot);
}

// dQ, fp32. The tile's K and V rows stream in halves (rows 0-63, 64-127) through two half
// buffers: the copy of one half runs while the other is computed. Two barriers per tile.

template <int D>
__global__ void __launch_bounds__(NT, 1) dq_f32_kernel(KArgs a) {
  constexpr int HB = 64 * D * 4;  // bytes of 64 rows of K or V
  __shared__ __attribute__((aligned(1024))) char h0[2 * HB];  // rows 0-63: K | V
  __shared__ __attribute__((aligned(1024))) char h1[2 * HB];  // rows 64-127: K | V
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i = lane & 31, g = lane >> 5;
  const Job j = decode_job(a);
  if (j.skip) return;  // an empty entry of the order table
  const uint32_t snb = (uint32_t)a.sn * 4;
  const rsrc_t rK = make_rsrc((const float*)a.k + j.base, a.slice_bytes);
  const rsrc_t rV = make_rsrc((const float*)a.v + j.base, a.slice_bytes);

  const int qrow = j.blk * BLK + 32 * w + i;
  f32x4 qf[D / 8], df[D / 8];
  load_frag_f32<D>(qf, make_rsrc((const float*)a.q + j.base, a.slice_bytes), qrow, snb, g);
  load_frag_f32<D>(df, make_rsrc((const float*)a.dout + j.obase, a.oslice_bytes), qrow, (uint32_t)a.osn * 4, g);
  float lse_t = 0.f, delta = 0.f;
  if (qrow < a.n) {
    lse_t = a.lse[stat_index(a, j, qrow)] * LOG2E;
    delta = a.delta[stat_index(a, j, qrow)];
  }
  F32Offsets<D> off;
  off.init(i, g);
  HalfDma<D> dma;
  dma.init(w, lane, snb, true);
  f32x16 acc[D / 32];
#pragma unroll
  for (int db = 0; db < D / 32; ++db) acc[db] = zero16();

  // Key group sb of the tile, from the half buffer holding it (local group sl = sb % 2).
  auto group = [&](int sb, int sl, const char* ldsK, const char* ldsV, u32x2 mb) {
    f32x16 s = zero16(), dp = zero16();
    f32x4 kx[D / 8], vx[D / 8];
#pragma unroll
    for (int u = 0; u < D / 8; ++u) {
      kx[u] = *(const f32x4*)(ldsK + off.row[u & 3] + off.row_imm(sl, u));
      vx[u] = *(const f32x4*)(ldsV + off.row[u & 3] + off.row_imm(sl, u));
    }
#pragma unroll
    for (int u = 0; u < D / 8; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        s = mfma_f32(kx[u][e], qf[u][e], s);
        dp = mfma_f32(vx[u][e], df[u][e], dp);
      }
    sched_reads_ahead<D / 8, 2, 8>();
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float p = fast_exp2(fmaf(s[r], a.c2, -lse_t));
      p = keep_or_zero(p, elem_keep(mb, sb, r));
      dp[r] = p * (dp[r] - delta);
    }
    float kt[16][D / 32];
#pragma unroll
    for (int r = 0; r < 16; ++r)
#pragma unroll
      for (int db = 0; db < D / 32; ++db) kt[r][db] = *(const float*)(ldsK + off.el[r & 3] + off.el_imm(sl, r, db));
#pragma unroll
    for (int r = 0; r < 16; ++r) {
#pragma unroll
      for (int db = 0; db < D / 32; ++db) acc[db] = mfma_f32(kt[r][db], dp[r], acc[db]);
    }
    sched_reads_ahead<16, D / 32, D / 32>();
  };

  int t0, t1;
  tile_range(a, j, t0, t1);
  uint32_t gcur = 0u;
  if (t0 < t1) {
    gcur = tile_groups(a, t0);
    const int kb = ((ci32_ptr)a.col)[t0];
    dma.issue(rK, h0, kb * BLK, snb, w, 0, any_rows(gcur));
    dma.issue(rV, h0 + HB, kb * BLK, snb, w, 0, any_rows(gcur));
  }
  for (int tt = t0; tt < t1; ++tt) {
    const int t = __builtin_amdgcn_readfirstlane(tt);
    const int kb = ((ci32_ptr)a.col)[t];
    const u32x2 mb = tile_bits(a, t, w, lane);
    const uint32_t gt = gcur;
    const uint32_t live = gt >> (4 * w) & 15u;  // key groups with p = 0 throughout are skipped
    wait_vmem();      // this wave's part of half 0 of tile t, and the mask bits
    __syncthreads();  // half 0 landed; every wave is done with half 1 of tile t - 1
    dma.issue(rK, h1, kb * BLK, snb, w, 1, any_rows(gt));
    dma.issue(rV, h1 + HB, kb * BLK, snb, w, 1, any_rows(gt));
    if (t + 1 < t1) gcur = tile_groups(a, t + 1);
    // Fenced, so that one group's reads and MFMAs do not overlap the next group's registers.
    __builtin_amdgcn_sched_barrier(0);
    if (live & 1u) group(0, 0, h0, h0 + HB, mb);
    __builtin_amdgcn_sched_barrier(0);
    if (live & 2u) group(1, 1, h0, h0 + HB, mb);
    __builtin_amdgcn_sched_barrier(0);
    wait_vmem();      // this wave's part of half 1
    __syncthreads();  // half 1 landed; every wave is done with half 0
    if (t + 1 < t1) {
      const int kbn = ((ci32_ptr)a.col)[t + 1];
      dma.issue(rK, h0, kbn * BLK, snb, w, 0, any_rows(gcur));
      dma.issue(rV, h0 + HB, kbn * BLK, snb, w, 0, any_rows(gcur));
    }
    __builtin_amdgcn_sched_barrier(0);
    if (live & 4u) group(2, 0, h1, h1 + HB, mb);
    __builtin_amdgcn_sched_barrier(0);
    if (live & 8u) group(3, 1, h1, h1 + HB, mb);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (j.part >= 0) {
    store_bwd_partial<D>(a, j, 32 * w + i, acc, 0, g);
    return;
  }
  store_acc_f32<D>(make_rsrc((float*)a.out0 + j.base, a.slice_bytes), qrow, snb, acc, a.scale, g);
}

// dQ, fp32, from the dS units of the float32 dK/dV kernels (the float32 dS exchange: written by
// dkv16_f32_kernel<true> at head_dim 128, dkv_f32_kernel<D, true> below it): per work
// item of the forward list, dQ^T += K^T dS^T over each wave's live 32 x 32 groups
// (pallas_attn.py:177-184 with dS from the dK/dV pass instead of recomputed). A unit is one
// group's dS, 4 KB, laid out so that lane L's B operands (query L % 32, key
// element_col(sb, r, L / 32) in register r) are its 16-byte chunks 64 k + L, k = 0..3: four
// 16-byte loads per lane and group, straight into the MFMA operands. No V, Q, dO or statistics
// are read and no S, dP or exponentials computed: a third of dq_f32_kernel's MFMAs.
//
// K rows stream in halves through two half buffers (32 KB each at D = 128), two workgroups per
// CU. A half's units are loaded together with its K rows, so the barrier that publishes the rows
// also covers the units.
template <int D>
__global__ void __launch_bounds__(NT, 2) dq_f32_ds_kernel(KArgs a) {
  constexpr int HB = 64 * D * 4;  // bytes of 64 rows of K
  __shared__ __attribute__((aligned(1024))) char h0[HB];  // rows 0-63
  __shared__ __attribute__((aligned(1024))) char h1[HB];  // rows 64-127
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i = lane & 31, g = lane >> 5;
  const Job j = decode_job(a);
  if (j.skip) return;  // an empty entry of the order table
  const uint32_t snb = (uint32_t)a.sn * 4;
  const rsrc_t rK = make_rsrc((const float*)a.k + j.base, a.slice_bytes);
  const rsrc_t rS = make_rsrc((const float*)a.ds + (int64_t)j.bh * (a.ds_slice_bytes >> 2), a.ds_slice_bytes);
  const int qrow = j.blk * BLK + 32 * w + i;
  F32Offsets<D> off;
  off.init(i, g);
  HalfDma<D> dma;
  dma.init(w, lane, snb, true);
  f32x16 acc[D / 32];
#pragma unroll
  for (int db = 0; db < D / 32; ++db) acc[db] = zero16();
  typedef const __attribute__((address_space(4))) int32_t* cmap_ptr;

  // This wave's units of tile half h (key groups 2h and 2h + 1: group bits 4w + 2h + x), numbered
  // from the tile's first unit by their rank among its 16 group bits. Each is read once:
  // non-temporal loads.
  auto load_units = [&](f32x4 (&dst)[2][4], uint32_t gw, uint32_t ub, int h) {
    const uint32_t b0 = 4u * (uint32_t)w + 2u * (uint32_t)h;
    uint32_t u = ub + (uint32_t)__builtin_popcount(gw & 0xffffu & ((1u << b0) - 1u));
#pragma unroll
    for (int x = 0; x < 2; ++x)
      if (gw >> (b0 + x) & 1u) {
#pragma unroll
        for (int k = 0; k < 4; ++k)
          // The unit's offset in the per-lane offset: checked against the slice size.
          dst[x][k] = __builtin_bit_cast(
              f32x4, __builtin_amdgcn_raw_buffer_load_b128(rS, (int)(16u * (64 * k + lane) + u * 4096u), 0, 2));
        ++u;
      }
  };
  // Key group sl of the half buffer ldsK, with its unit d. hv: the group's 16-key halves with a
  // valid element for this wave (bit h: registers 8 h .. 8 h + 7 of the unit); a clear half has
  // dS = 0 and skips its reads and MFMAs.
  auto group = [&](int sl, const char* ldsK, const f32x4 (&d)[4], uint32_t hv) {
#pragma unroll
    for (int h = 0; h < 2; ++h)
      if (hv >> h & 1u) {
        float kt[8][D / 32];
#pragma unroll
        for (int x = 0; x < 8; ++x)
#pragma unroll
          for (int db = 0; db < D / 32; ++db) {
            const int r = 8 * h + x;
            kt[x][db] = *(const float*)(ldsK + off.el[r & 3] + off.el_imm(sl, r, db));
          }
#pragma unroll
        for (int x = 0; x < 8; ++x) {
          const int r = 8 * h + x;
#pragma unroll
          for (int db = 0; db < D / 32; ++db) acc[db] = mfma_f32(kt[x][db], d[r >> 2][r & 3], acc[db]);
        }
        sched_reads_ahead<8, D / 32, D / 32>();
      }
  };

  int t0, t1;
  tile_range(a, j, t0, t1);
  f32x4 dsA[2][4], dsB[2][4];  // units of the current tile's half 0 and half 1
  uint32_t gcur = 0u, ucur = 0u;
  if (t0 < t1) {
    gcur = tile_groups(a, t0);
    ucur = (uint32_t)((cmap_ptr)a.ubase)[t0];
    dma.issue(rK, h0, ((ci32_ptr)a.col)[t0] * BLK, snb, w, 0, any_rows(gcur));
    load_units(dsA, gcur, ucur, 0);
  }
  for (int tt = t0; tt < t1; ++tt) {
    const int t = __builtin_amdgcn_readfirstlane(tt);
    const int kb = ((ci32_ptr)a.col)[t];
    const uint32_t gt = gcur, ut = ucur;
    const uint32_t live = gt >> (4 * w) & 15u;
    const uint32_t hw = tile_halves(a, t) >> (8 * w) & 0xffu;  // bit 2 sb + h: live 16-key halves
    wait_vmem();      // this wave's part of half 0 of tile t and its units
    __syncthreads();  // half 0 landed; every wave is done with half 1 of tile t - 1
    dma.issue(rK, h1, kb * BLK, snb, w, 1, any_rows(gt));
    load_units(dsB, gt, ut, 1);
    if (t + 1 < t1) {
      gcur = tile_groups(a, t + 1);
      ucur = (uint32_t)((cmap_ptr)a.ubase)[t + 1];
    }
    __builtin_amdgcn_sched_barrier(0);
    if (live & 1u) group(0, h0, dsA[0], hw & 3u);
    __builtin_amdgcn_sched_barrier(0);
    if (live & 2u) group(1, h0, dsA[1], hw >> 2 & 3u);
    __builtin_amdgcn_sched_barrier(0);
    wait_vmem();      // this wave's part of half 1 and its units
    __syncthreads();  // half 1 landed; every wave is done with half 0
    if (t + 1 < t1) {
      dma.issue(rK, h0, ((ci32_ptr)a.col)[t + 1] * BLK, snb, w, 0, any_rows(gcur));
      load_units(dsA, gcur, ucur, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (live & 4u) group(0, h1, dsB[0], hw >> 4 & 3u);
    __builtin_amdgcn_sched_barrier(0);
    if (live & 8u) group(1, h1, dsB[1], hw >> 6 & 3u);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (j.part >= 0) {
    store_bwd_partial<D>(a, j, 32 * w + i, acc, 0, g);
    return;
  }
  store_acc_f32<D>(make_rsrc((float*)a.out0 + j.base, a.slice_bytes), qrow, snb, acc, a.scale, g);
}

// dK/dV, fp32, head_dim 32 and 64 (head_dim 128 runs dkv16_f32_kernel). The tile's Q and dO
// rows, and their lse and delta, stream in halves through two half buffers as in dQ.
//
// With DS (the float32 dS exchange), each group's dS also goes to HBM as one 4 KB unit in
// dq_f32_ds_kernel's operand layout. This lane holds dS of key 32w + i and query
// element_col(sb, r, g) in register r; in the unit that value belongs to dQ lane
// (query, (key % 32 / 8) % 2), register 8 (key % 32 / 16) + key % 8, so each of the 16 stores
// has a per-lane offset fixed at the start plus an immediate per register. Units are numbered
// over the forward list by the rank of group bit 4 sb + w (query group sb, key group w) in the
// forward tile's group word; tmap gives that word and the tile's first unit.
template <int D, bool DS = false>
__global__ void __launch_bounds__(NT, 1) dkv_f32_kernel(KArgs a) {
  constexpr int HB = 64 * D * 4;  // bytes of 64 rows of Q or dO
  // rows 0-63 (h0) and 64-127 (h1): Q | dO | lse * log2(e) [64] | delta [64]
  __shared__ __attribute__((aligned(1024))) char h0[2 * HB + 512];
  __shared__ __attribute__((aligned(1024))) char h1[2 * HB + 512];
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i = lane & 31, g = lane >> 5;
  const Job j = decode_job(a);
  if (j.skip) return;  // an empty entry of the order table
  const uint32_t snb = (uint32_t)a.sn * 4;
  const rsrc_t rQ = make_rsrc((const float*)a.q + j.base, a.slice_bytes);
  const rsrc_t rO = make_rsrc((const float*)a.dout + j.obase, a.oslice_bytes);
  const uint32_t osnb = (uint32_t)a.osn * 4;
  const rsrc_t rL = make_rsrc(a.lse + stat_index(a, j, 0), (uint32_t)a.n * 4);
  const rsrc_t rD = make_rsrc(a.delta + stat_index(a, j, 0), (uint32_t)a.n * 4);

  const int krow = j.blk * BLK + 32 * w + i;
  f32x4 kf[D / 8], vf[D / 8];
  load_frag_f32<D>(kf, make_rsrc((const float*)a.k + j.base, a.slice_bytes), krow, snb, g);
  load_frag_f32<D>(vf, make_rsrc((const float*)a.v + j.base, a.slice_bytes), krow, snb, g);
  F32Offsets<D> off;
  off.init(i, g);
  HalfDma<D> dmaQ, dmaO;
  dmaQ.init(w, lane, snb, true);
  dmaO.init(w, lane, osnb, true);
  f32x16 dk[D / 32], dv[D / 32];
#pragma unroll
  for (int db = 0; db < D / 32; ++db) {
    dk[db] = zero16();
    dv[db] = zero16();
  }
  // dS exchange: this (batch, head)'s unit slice (a plain global pointer: a buffer resource's
  // four SGPRs would push this kernel past its SGPR budget), this lane's offset in a unit, and
  // the current tile's first unit and group word.
  char* dsb = nullptr;
  uint32_t dsl = 0u, ubc = 0u, gfc = 0u;
  typedef const __attribute__((address_space(4))) uint32_t* cmap_ptr;
  if constexpr (DS) {
    dsb = (char*)a.ds + (int64_t)j.bh * a.ds_slice_bytes;
    const int tk = (i >> 3) & 1, tr = 8 * (i >> 4) + (i & 7);
    dsl = (uint32_t)((64 * (tr >> 2) + 32 * tk + 8 * g) * 16 + 4 * (tr & 3));
  }

  // Half h of query block qb: the Q and dO rows (live groups only) and, by wave 0, the 64 rows'
  // lse and delta (4 bytes per lane; rows past n read zeros).
  auto copy_half = [&](char* hb, int qb, int h, uint32_t live) {
    dmaQ.issue(rQ, hb, qb * BLK, snb, w, h, live);
    dmaO.issue(rO, hb + HB, qb * BLK, osnb, w, h, live);
    if (w == 0) {
      const int so = (qb * BLK + 64 * h + lane) * 4;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rL, (__attribute__((address_space(3))) void*)(hb + 2 * HB), 4, so, 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rD, (__attribute__((address_space(3))) void*)(hb + 2 * HB + 256), 4, so, 0, 0, 0);
    }
  };
  // After the copy of a half landed: lse -> lse * log2(e), the form the exponent takes.
  auto scale_lse = [&](char* hb) {
    if (w == 0 && lane < 16) {
      f32x4* x = (f32x4*)(hb + 2 * HB + 16 * lane);
      *x = *x * LOG2E;
    }
  };
  // Query group sb of the tile, from the half buffer holding it (local group sl = sb % 2).
  auto group = [&](int sb, int sl, const char* hb, u32x2 mb) {
    const char* ldsQ = hb;
    const char* ldsO = hb + HB;
    const float* ldsL = (const float*)(hb + 2 * HB);
    const float* ldsDl = ldsL + 64;
    f32x16 s = zero16(), dp;
#pragma unroll
    for (int r = 0; r < 16; ++r) dp[r] = -ldsDl[element_col(sl, r, g)];  // dP^T - delta accumulates directly
    f32x4 qx[D / 8], ox[D / 8];
#pragma unroll
    for (int u = 0; u < D / 8; ++u) {
      qx[u] = *(const f32x4*)(ldsQ + off.row[u & 3] + off.row_imm(sl, u));
      ox[u] = *(const f32x4*)(ldsO + off.row[u & 3] + off.row_imm(sl, u));
    }
#pragma unroll
    for (int u = 0; u < D / 8; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        s = mfma_f32(qx[u][e], kf[u][e], s);
        dp = mfma_f32(ox[u][e], vf[u][e], dp);
      }
    sched_reads_ahead<D / 8, 2, 8>();
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float p = fast_exp2(fmaf(s[r], a.c2, -ldsL[element_col(sl, r, g)]));
      p = keep_or_zero(p, elem_keep(mb, sb, r));
      s[r] = p;
      dp[r] = p * dp[r];
    }
    if constexpr (DS) {
      const uint32_t bit = 4u * (uint32_t)sb + (uint32_t)w;
      const uint32_t so = (ubc + (uint32_t)__builtin_popcount(gfc & 0xffffu & ((1u << bit) - 1u))) * 4096u;
      // A plain pointer has no range check: store only a unit the map has, inside the slice (a
      // map of other lists cannot write outside the buffer).
      if ((gfc >> bit & 1u) && so + 4096u <= a.ds_slice_bytes) {
        float* u = (float*)(dsb + (so + dsl));
#pragma unroll
        for (int r = 0; r < 16; ++r) u[4 * (16 * (r >> 3) + (r & 7))] = dp[r];
      }
    }
    float ot[16][D / 32], qt[16][D / 32];
#pragma unroll
    for (int r = 0; r < 16; ++r)
#pragma unroll
      for (int db = 0; db < D / 32; ++db) {
        ot[r][db] = *(const float*)(ldsO + off.el[r & 3] + off.el_imm(sl, r, db));
        qt[r][db] = *(const float*)(ldsQ + off.el[r & 3] + off.el_imm(sl, r, db));
      }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
#pragma unroll
      for (int db = 0; db < D / 32; ++db) {
        dv[db] = mfma_f32(ot[r][db], s[r], dv[db]);
        dk[db] = mfma_f32(qt[r][db], dp[r], dk[db]);
      }
    }
    sched_reads_ahead<16, 2 * (D / 32), 2 * (D / 32)>();
  };

  int t0, t1;
  tile_range(a, j, t0, t1);
  uint32_t gcur = 0u;
  if (t0 < t1) {
    gcur = tile_groups(a, t0);
    copy_half(h0, ((ci32_ptr)a.col)[t0], 0, any_rows(gcur));
  }
  for (int tt = t0; tt < t1; ++tt) {
    const int t = __builtin_amdgcn_readfirstlane(tt);
    const int qb = ((ci32_ptr)a.col)[t];
    const u32x2 mb = tile_bits(a, t, w, lane);
    const uint32_t gt = gcur;
    const uint32_t live = gt >> (4 * w) & 15u;  // query groups with p = 0 throughout are skipped
    if constexpr (DS) {
      ubc = ((cmap_ptr)a.tmap)[2 * t];
      gfc = ((cmap_ptr)a.tmap)[2 * t + 1];
    }
    wait_vmem();  // this wave's part of half 0 of tile t, and the mask bits
    scale_lse(h0);
    __syncthreads();  // half 0 landed; every wave is done with half 1 of tile t - 1
    copy_half(h1, qb, 1, any_rows(gt));
    if (t + 1 < t1) gcur = tile_groups(a, t + 1);
    // Fenced, so that one group's reads and MFMAs do not overlap the next group's registers.
    __builtin_amdgcn_sched_barrier(0);
    if (live & 1u) group(0, 0, h0, mb);
    __builtin_amdgcn_sched_barrier(0);
    if (live & 2u) group(1, 1, h0, mb);
    __builtin_amdgcn_sched_barrier(0);
    wait_vmem();  // this wave's part of half 1
    scale_lse(h1);
    __syncthreads();  // half 1 landed; every wave is done with half 0
    if (t + 1 < t1) copy_half(h0, ((ci32_ptr)a.col)[t + 1], 0, any_rows(gcur));
    __builtin_amdgcn_sched_barrier(0);
    if (live & 4u) group(2, 0, h1, mb);
    __builtin_amdgcn_sched_barrier(0);
    if (live & 8u) group(3, 1, h1, mb);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (j.part >= 0) {
    store_bwd_partial<D>(a, j, 32 * w + i, dk, 0, g);
    store_bwd_partial<D>(a, j, 32 * w + i, dv, 1, g);
    return;
  }
  store_acc_f32<D>(make_rsrc((float*)a.out0 + j.base, a.slice_bytes), krow, snb, dk, a.scale, g);
  store_acc_f32<D>(make_rsrc((float*)a.out1 + j.base, a.slice_bytes), krow, snb, dv, 1.f, g);
}

// ------------------------------------------------------------------------------------------
// dK/dV, fp32, head_dim 128, 16 keys per wave (V_MFMA_F32_16X16X4F32): a wave's K and V rows (64
// registers) and dK^T, dV^T (64) leave room for a second wave per SIMD, twice dkv_f32_kernel's
// waves per CU. Each work item's 128 keys are split between two 4-wave workgroups of 64 keys (78
// KB of LDS each), two per CU: each streams only the query groups its own keys need, and the two
// meet at barriers of their own, so one's waiting waves leave their SIMDs to the other's. The two
// halves of an item sit on the same XCD and share its L2 for the Q and dO groups both read.
//
// The k order of the first contractions is permuted so that each lane's fragment is contiguous:
// k-step s of lane group g (= lane / 16) contracts column 32 g + s, so lane (key l % 16, g) holds
// K and V columns 32 g .. 32 g + 31 of its key, and one 16-byte row read of a Q or dO row gives
// the A operands of four k-steps. The accumulator layout is the bf16 16-key kernel's: lane
// (key l % 16, g) holds S and dP of queries 16 m + 4 g + r. P and dS are then the B operands of
// dV^T += dO^T P and dK^T += Q^T dS with query 16 m + 4 g + r as step (m, r), and the A operands
// are single dO / Q elements, read straight from the row-major tile.
//
// Tiles: the transposed list's (tile, query group) steps stream the group's Q and dO rows and its
// statistics through two group buffers. Rows are padded to 528 bytes (16 bytes over a row), so
// every LDS address is a per-lane base plus an immediate and both read patterns spread over the
// banks without a swizzle: 16 lanes of a row read cover rows t .. t + 15 at one column (16 t bytes
// apart modulo the 256-byte bank line), and the 64 lanes of an element read cover rows 4 g + r at
// 16 columns (64 g bytes apart). A padded row is one LDS DMA instruction of 32 lanes.
//
// dS (DS): the float32 exchange's 4 KB units, written by the two waves of a 32-key group: the wave
// of 16-key group kg writes dQ registers 8 (kg % 2) .. + 7 of every dQ lane (chunks 2 (kg % 2) and
// 2 (kg % 2) + 1) through its own LDS stage ([query][16 keys] fp32, 80-byte rows). A wave whose
// 16 keys have no valid element in a unit the map has writes zeros for its chunks.
constexpr int kRowPad = 4 * 128 + 16;  // padded LDS row of a head_dim 128 fp32 tile
constexpr uint32_t kPastEndF = 0x7FFFFFF0u;  // a buffer offset past every slice: reads zeros

__device__ __forceinline__ f32x4 mfma16f(float a, float b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

template <bool DS>
__global__ void __launch_bounds__(256, 2) dkv16_f32_kernel(KArgs a) {
  constexpr int D = 128;
  constexpr int RB = kRowPad;
  constexpr int PB = 32 * RB;  // one plane: 32 padded rows
  constexpr int SB = 2 * PB;   // Q | dO | -lse/scale [32], 0 [32] | -delta [32], 0 [32]
  constexpr int NB = D / 16;   // 16-column blocks of dK^T and dV^T
  constexpr int SROW = 80;
  __shared__ __attribute__((aligned(1024))) char gb0[SB + 512];
  __shared__ __attribute__((aligned(1024))) char gb1[SB + 512];
  __shared__ __attribute__((aligned(16))) char stage[DS ? 4 * 32 * SROW : 16];
  typedef const __attribute__((address_space(3))) f32x4* cf4;
  // Element reads are volatile so that the compiler does not pair them into ds_read2_b32 (rows r
  // and r + 1, or column blocks n and n + 1): with single reads the kernel measured 6% faster.
  typedef const volatile __attribute__((address_space(3))) float* cv1;
  typedef const __attribute__((address_space(4))) uint32_t* cmap_ptr;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, t16 = lane & 15;
  // Two workgroups per work item, one per 64-key half of the block, on the same XCD (workgroup
  // ids 16 i + x and 16 i + 8 + x): pid = 8 i + x is the item's id as decode_job numbers them.
  const int half = (int)(blockIdx.x >> 3) & 1;
  const int pid = (int)(((blockIdx.x >> 4) << 3) | (blockIdx.x & 7));
  if (pid >= job_count(a)) return;
  const Job j = decode_job(a, pid);
  if (j.skip) return;  // an empty entry of the order table
  const int kg = 4 * half + wid;  // this wave's 16-key group of the block
  const uint32_t snb = (uint32_t)a.sn * 4, osnb = (uint32_t)a.osn * 4;
  const rsrc_t rQ = make_rsrc((const float*)a.q + j.base, a.slice_bytes);
  const rsrc_t rO = make_rsrc((const float*)a.dout + j.obase, a.oslice_bytes);
  const rsrc_t rL = make_rsrc(a.lse + stat_index(a, j, 0), (uint32_t)a.n * 4);
  const rsrc_t rD = make_rsrc(a.delta + stat_index(a, j, 0), (uint32_t)a.n * 4);
  const rsrc_t rS = make_rsrc(DS ? (const void*)(a.ds + (int64_t)j.bh * (a.ds_slice_bytes >> 1)) : (const void*)a.q,
                              DS ? a.ds_slice_bytes : 0u);
  const int krow = j.blk * BLK + 16 * kg + t16;
  // K and V of this lane's key: kf[u][e] = column 32 g + 4 u + e (k-step 4 u + e).
  f32x4 kf[8], vf[8];
  {
    const rsrc_t rK = make_rsrc((const float*)a.k + j.base, a.slice_bytes);
    const rsrc_t rV = make_rsrc((const float*)a.v + j.base, a.slice_bytes);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const uint32_t off = (uint32_t)krow * snb + (uint32_t)(128 * g + 16 * u);
      kf[u] = __builtin_bit_cast(f32x4, bload16(rK, off));
      vf[u] = __builtin_bit_cast(f32x4, bload16(rV, off));
    }
  }
  // Per-lane LDS bases: row reads (row t16, columns 32 g ..) and element reads (row 4 g, column
  // t16); the loop indexes add immediates.
  const uint32_t rbase = (uint32_t)(t16 * RB + 128 * g);
  const uint32_t ebase = (uint32_t)(4 * g * RB + 4 * t16);
  f32x4 dk[NB], dv[NB];
#pragma unroll
  for (int n = 0; n < NB; ++n) {
    dk[n] = f32x4{0.f, 0.f, 0.f, 0.f};
    dv[n] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const uint64_t* mword = key_mask_words(a, kg, g, t16);
  const int mshift = 4 * (g & 1);
  lds_char* stw = (lds_char*)stage + wid * 32 * SROW;

  // The dS chunks of a unit: `have` false writes zeros.
  auto store_chunks = [&](bool have, const float (&ds)[8], uint32_t u) {
    const int i = lane & 31, gq = lane >> 5;
    u32x4 y[2] = {u32x4{0u, 0u, 0u, 0u}, u32x4{0u, 0u, 0u, 0u}};
    if (have) {
      asm volatile("" ::: "memory");
#pragma unroll
      for (int e = 0; e < 8; ++e)
        *(__attribute__((address_space(3))) float*)(stw + (16 * (e >> 2) + 4 * g + (e & 3)) * SROW + 4 * t16) = ds[e];
      asm volatile("" ::: "memory");
#pragma unroll
      for (int h = 0; h < 2; ++h)
        y[h] = *(const __attribute__((address_space(3))) u32x4*)(stw + i * SROW + 32 * gq + 16 * h);
      asm volatile("" ::: "memory");
    }
#pragma unroll
    for (int h = 0; h < 2; ++h)  // the unit's offset in the per-lane offset: checked against the slice size
      __builtin_amdgcn_raw_buffer_store_b128(y[h], rS, (int)(16u * (64 * (2 * (wid & 1) + h) + lane) + u * 4096u), 0, 2);
  };

  // Unit: query group c of the group buffer buf (mask word mw of this lane); dS into ds. hm is the
  // set of 16-query halves (bit m: queries 16 m .. 16 m + 15) in which these 16 keys have a valid
  // element (wave-uniform). A half without one would add exact zeros: its S, dP, dV and dK MFMAs
  // are skipped by uniform branches and its dS stays zero. The reads are not: one code path keeps
  // dK^T / dV^T in the same registers whichever halves run.
  auto unit = [&](int c, const lds_char* buf, uint64_t mw, uint32_t hm, float (&ds)[8]) {
    const lds_char* lq = buf;
    const lds_char* lo = buf + PB;
    f32x4 sa[2], da[2];
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      sa[m] = *(cf4)(buf + SB + 4 * (16 * m + 4 * g));
      da[m] = *(cf4)(buf + SB + 256 + 4 * (16 * m + 4 * g));
    }
    // S and dP: the Q and dO row reads of the next (row read u, query half m) go out before this
    // pair's eight MFMAs.
    auto rows = [&](f32x4 (&x)[2], int it) {
      const uint32_t o = rbase + (uint32_t)(16 * (it >> 1) + 16 * (it & 1) * RB);
      x[0] = *(cf4)(lq + o);
      x[1] = *(cf4)(lo + o);
    };
    f32x4 rd[2][2];
    rows(rd[0], 0);
    __builtin_amdgcn_s_setprio(1);  // MFMA phases at issue priority 1, the exponentials at 0
#pragma unroll
    for (int it = 0; it < 16; ++it) {
      if (it + 1 < 16) rows(rd[(it + 1) & 1], it + 1);
      __builtin_amdgcn_sched_barrier(0);
      const int u = it >> 1, m = it & 1;
      if (hm >> m & 1u) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          sa[m] = mfma16f(rd[it & 1][0][e], kf[u][e], sa[m]);
          da[m] = mfma16f(rd[it & 1][1][e], vf[u][e], da[m]);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    __builtin_amdgcn_s_setprio(0);
    float p[8];
    const uint32_t w32 = (uint32_t)(mw >> (32 * (c >> 1)));
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float se = e < 4 ? sa[0][e & 3] : sa[1][e & 3];
      const float de = e < 4 ? da[0][e & 3] : da[1][e & 3];
      // A skipped half's bits are all clear: p = 0 there, whatever its accumulators hold.
      const float pe = keep_or_zero(fast_exp2(se * a.c2),
                                    __builtin_amdgcn_sbfe(w32, (uint32_t)(16 * (c & 1) + 8 * (e >> 2) + (e & 3)), 1u));
      p[e] = pe;
      ds[e] = pe * de;
    }
    // dV^T and dK^T by 16-column block n; the block's 16 element reads go out before the previous
    // block's MFMAs.
    auto els = [&](float (&x)[16], int n) {
#pragma unroll
      for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const uint32_t o = ebase + (uint32_t)((16 * m + r) * RB + 64 * n);
          x[8 * m + 2 * r] = *(cv1)(lo + o);
          x[8 * m + 2 * r + 1] = *(cv1)(lq + o);
        }
    };
    float ex[2][16];
    els(ex[0], 0);
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int n = 0; n < NB; ++n) {
      if (n + 1 < NB) els(ex[(n + 1) & 1], n + 1);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int m = 0; m < 2; ++m)
        if (hm >> m & 1u) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            dv[n] = mfma16f(ex[n & 1][8 * m + 2 * r], p[4 * m + r], dv[n]);
            dk[n] = mfma16f(ex[n & 1][8 * m + 2 * r + 1], ds[4 * m + r], dk[n]);
          }
        }
      __builtin_amdgcn_sched_barrier(0);
    }
    __builtin_amdgcn_s_setprio(0);
  };

  int t0, t1;
  tile_range(a, j, t0, t1);
  int ti = t0 - 1;
  uint32_t rem = 0u;
  auto take = [&](int& t, int& c) -> bool {
    while (rem == 0u) {
      if (++ti >= t1) return false;
      // query groups with a valid element for this half's keys (32-key groups 2 half, 2 half + 1)
      const uint32_t tg = tile_groups(a, ti) >> (8 * half);
      rem = (tg | tg >> 4) & 15u;
    }
    t = ti;
    c = __builtin_ctz(rem);
    rem &= rem - 1u;
    return true;
  };
  // Rows row0 .. row0 + 31 of Q (plane 0) and dO (plane 1), one padded row per instruction: wave w
  // copies rows w + 4 m' of both planes with lanes 0-31 (16 bytes each); then, by wave 0, the
  // group's lse and delta (rows past n read zeros).
  auto copy = [&](lds_char* buf, int t, int c) {
    const int row0 = ((ci32_ptr)a.col)[t] * BLK + 32 * c;
    uint32_t base = (uint32_t)(uintptr_t)buf;
    asm volatile("" : "+s"(base));
    if (lane < 32) {
#pragma unroll
      for (int m = 0; m < 16; ++m) {
        const int plane = m >> 3, row = wid + 4 * (m & 7);
        const uint32_t src = (uint32_t)(row0 + row) * (plane ? osnb : snb) + (uint32_t)(16 * lane);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            plane ? rO : rQ, (__attribute__((address_space(3))) void*)(uintptr_t)(base + (uint32_t)(plane * PB + row * RB)),
            16, (int)src, 0, 0, 0);
      }
    }
    if (wid == 0) {
      const int so = lane < 32 ? (row0 + lane) * 4 : (int)kPastEndF;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rL, (__attribute__((address_space(3))) void*)(buf + SB), 4, so, 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rD, (__attribute__((address_space(3))) void*)(buf + SB + 256), 4, so, 0,
                                               0, 0);
    }
  };
  lds_char* b0 = (lds_char*)gb0;
  lds_char* b1 = (lds_char*)gb1;
  int tc = 0, cc = 0, tn = 0, cn = 0;
  bool vc = take(tc, cc), vn = false;
  uint64_t mwc = 0, mwn = 0;
  if (vc) {
    copy(b0, tc, cc);
    mwc = mword[(int64_t)tc * 256];
    vn = take(tn, cn);
  }
  auto step = [&](lds_char* cur, lds_char* nxt) {
    wait_vmem();  // this wave's part of the current step (wave 0: the statistics) and its mask word
    if (wid == 0 && lane < 16) {
      // lse -> -lse / scale and delta -> -delta: the initial values of the S and dP accumulators.
      __attribute__((address_space(3))) f32x4* x =
          (__attribute__((address_space(3))) f32x4*)(cur + SB + (lane < 8 ? 16 * lane : 256 + 16 * (lane - 8)));
      float mul = lane < 8 ? a.nlse_mul : -1.f;
      asm volatile("" : "+v"(mul));
      *x = *x * mul;
    }
    __syncthreads();  // the step landed; every wave is done with the previous step's buffer
    if (vn) {
      copy(nxt, tn, cn);
      mwn = tn != tc ? mword[(int64_t)tn * 256] : mwc;
    }
    // The 16-query halves of group cc in which the wave's 16 keys have a valid element: some
    // lane's bits 16 cc + 8 m + r (shifted by 4 (g % 2)) are set.
    const uint64_t mw = mwc >> mshift;
    const uint32_t b8 = (uint32_t)(mw >> (16 * cc));
    const bool live0 = __builtin_amdgcn_ballot_w64((b8 & 0x000Fu) != 0u) != 0u;
    const bool live1 = __builtin_amdgcn_ballot_w64((b8 & 0x0F00u) != 0u) != 0u;
    const bool live = live0 || live1;
    bool have_unit = false;
    uint32_t u_idx = 0u;
    if constexpr (DS) {
      const uint32_t ub = ((cmap_ptr)a.tmap)[2 * tc];
      const uint32_t gw = ((cmap_ptr)a.tmap)[2 * tc + 1];
      const uint32_t bit = 4u * (uint32_t)cc + (uint32_t)(kg >> 1);
      have_unit = (gw >> bit & 1u) != 0u;
      u_idx = ub + (uint32_t)__builtin_popcount(gw & 0xffffu & ((1u << bit) - 1u));
    }
    // One store path after the unit (dS of a unit the map has, zeros where these 16 keys have no
    // valid element): a store inside the unit's branch, and another beside it, made the register
    // allocator place dK^T / dV^T differently on each path and copy them (64 VGPRs) every step.
    float ds[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (live) unit(cc, cur, mw, (live0 ? 1u : 0u) | (live1 ? 2u : 0u), ds);
    if constexpr (DS) {
      if (have_unit) store_chunks(live, ds, u_idx);
    }
    tc = tn;
    cc = cn;
    mwc = mwn;
    vc = vn;
    vn = vc && take(tn, cn);
  };
  while (vc) {
    step(b0, b1);
    if (!vc) break;
    step(b1, b0);
  }
  if (j.part >= 0) {
    const rsrc_t r = part_slot<D>(a, j);
    const int prow = 16 * kg + t16;
#pragma unroll
    for (int n = 0; n < NB; ++n) {
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, dk[n]), r,
                                             (int)((uint32_t)(prow * D + 16 * n + 4 * g) * 4), 0, 0);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, dv[n]), r,
                                             (int)((uint32_t)((128 + prow) * D + 16 * n + 4 * g) * 4), 0, 0);
    }
    return;
  }
  const rsrc_t rdk = make_rsrc((float*)a.out0 + j.base, a.slice_bytes);
  const rsrc_t rdv = make_rsrc((float*)a.out1 + j.base, a.slice_bytes);
#pragma unroll
  for (int n = 0; n < NB; ++n) {
    const uint32_t off = (uint32_t)krow * snb + (uint32_t)(4 * (16 * n + 4 * g));
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, dk[n] * a.scale), rdk, (int)off, 0, 0);
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, dv[n]), rdv, (int)off, 0, 0);
  }
}

// ------------------------------------------------------------------------------------------
// delta = rowsum(o * dout) (pallas_attn.py:278): L lanes per (batch, row, head), 16 B per lane.
// The grid is (row blocks x batch), flattened into x (a y extent would cap batch at 65,535): each
// workgroup takes one row block of one batch member, each lane group one row, and walks its heads, four at a
// time with every load issued before the first sum, so consecutive lane groups read consecutive
// rows and no lane divides by a runtime size (the earlier per-lane 64-bit index divisions took
// about 1,000 VALU instructions per four rows). Measured at 4.9-5.4 TB/s of O and dO reads
// (configurations 3 and 4), about what a streaming read reaches on MI355X. The sum of one row is
// formed in the same order as one row per lane group would form it.
template <typename T, int D>
__global__ void __launch_bounds__(NT) delta_kernel(KArgs a) {
  constexpr int EPC = 16 / (int)sizeof(T);
  constexpr int L = D / EPC;
  constexpr int GROUPS = NT / L;  // rows per workgroup
  constexpr int HB = 4;           // heads in flight per lane
  const int part = (int)(threadIdx.x % L);
  const int nrb = (a.n + GROUPS - 1) / GROUPS;  // row blocks per batch member (uniform)
  const int b = (int)blockIdx.x / nrb;
  const int row = ((int)blockIdx.x - b * nrb) * GROUPS + (int)(threadIdx.x / L);
  const bool ok = row < a.n;
  const int64_t rbase = (int64_t)b * a.osb + (int64_t)row * a.osn + part * EPC;
  for (int h0 = 0; h0 < a.heads; h0 += HB) {
    u32x4 x[HB], y[HB];
#pragma unroll
    for (int k = 0; k < HB; ++k) {
      x[k] = y[k] = u32x4{0u, 0u, 0u, 0u};
      if (ok && h0 + k < a.heads) {
        const int64_t off = rbase + (int64_t)(h0 + k) * a.osh;
        x[k] = *(const u32x4*)((const T*)a.o + off);
        y[k] = *(const u32x4*)((const T*)a.dout + off);
      }
    }
#pragma unroll
    for (int k = 0; k < HB; ++k) {
      float sum = 0.f;
      if constexpr (sizeof(T) == 4) {
        const f32x4 fx = __builtin_bit_cast(f32x4, x[k]), fy = __builtin_bit_cast(f32x4, y[k]);
#pragma unroll
        for (int e = 0; e < 4; ++e) sum += fx[e] * fy[e];
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          sum += __uint_as_float(x[k][e] << 16) * __uint_as_float(y[k][e] << 16);
          sum += __uint_as_float(x[k][e] & 0xffff0000u) * __uint_as_float(y[k][e] & 0xffff0000u);
        }
      }
#pragma unroll
      for (int o = L / 2; o > 0; o >>= 1) sum += __shfl_xor(sum, o);
      if (ok && h0 + k < a.heads && part == 0) a.lse_out[((int64_t)b * a.heads + h0 + k) * a.n + row] = sum;
    }
  }
}

// Grid of the delta kernel for a call: row blocks x batch members.
template <typename T, int D>
dim3 delta_grid(const KArgs& a) {
  constexpr int rows = NT / (D / (16 / (int)sizeof(T)));
  return dim3((unsigned)(((int64_t)a.n + rows - 1) / rows * a.batch));
}

template <int D>
hipError_t launch_d(Kind kind, const KArgs& a, hipStream_t stream) {
  const dim3 block(NT);
  if (kind == Kind::kDelta) {
    hipLaunchKernelGGL((delta_kernel<float, D>), (delta_grid<float, D>(a)), block, 0, stream, a);
    return hipGetLastError();
  }
  const dim3 grid((unsigned)job_count(a));
  // dkv16_f32_kernel: two workgroups per item, laid out in blocks of 16 ids (8 items x 2 halves).
  const dim3 grid2(16u * (((unsigned)job_count(a) + 7u) / 8u));
  switch (kind) {
    case Kind::kFwd: hipLaunchKernelGGL(fwd_f32g_kernel<D>, grid, block, 0, stream, a); break;
    case Kind::kDq: hipLaunchKernelGGL(dq_f32_kernel<D>, grid, block, 0, stream, a); break;
    case Kind::kDkv:
      if constexpr (D == 128) hipLaunchKernelGGL((dkv16_f32_kernel<false>), grid2, dim3(256), 0, stream, a);
      else hipLaunchKernelGGL((dkv_f32_kernel<D, false>), grid, block, 0, stream, a);
      break;
    case Kind::kDkvDs:
      if constexpr (D == 128) hipLaunchKernelGGL((dkv16_f32_kernel<true>), grid2, dim3(256), 0, stream, a);
      else hipLaunchKernelGGL((dkv_f32_kernel<D, true>), grid, block, 0, stream, a);
      break;
    case Kind::kDqDs: hipLaunchKernelGGL(dq_f32_ds_kernel<D>, grid, block, 0, stream, a); break;
    default: break;
  }
  return hipGetLastError();
}

template <int D>
hipError_t launch_delta_bf16_d(const KArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL((delta_kernel<uint16_t, D>), (delta_grid<uint16_t, D>(a)), dim3(NT), 0, stream, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_f32(Kind kind, int head_dim, const KArgs& a, hipStream_t stream) {
  switch (head_dim) {
    case 32: return launch_d<32>(kind, a, stream);
    case 64: return launch_d<64>(kind, a, stream);
    case 128: return launch_d<128>(kind, a, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_delta_bf16(int head_dim, const KArgs& a, hipStream_t stream) {
  switch (head_dim) {
    case 32: return launch_delta_bf16_d<32>(a, stream);
    case 64: return launch_delta_bf16_d<64>(a, stream);
    case 128: return launch_delta_bf16_d<128>(a, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace fwn
