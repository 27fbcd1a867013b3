// bfloat16 attention kernels for gfx950: forward, dQ, dK/dV (V_MFMA_F32_32X32X16_BF16, fp32
// accumulation, fp32 softmax statistics).
//
// Tiles live in LDS only row-major ([128 rows][D], 16-byte chunks XOR-swizzled) and are copied
// there by the buffer unit (buffer_load ... lds: each wave-wide instruction writes 1 KB, lane l at
// M0 + 16*l, from any per-lane global address), with no staging registers; the next tile streams
// in while the current one is computed (the forward per operand, the backward kernels into a
// second buffer). Both contractions read their A operands from the same copy:
//   - row reads (ds_read_b128) of the sigma-ordered rows for the first contraction;
//   - transpose reads (ds_read_b64_tr_b16) for the second: within each 16-lane group, lane 4e+q
//     addresses 4 consecutive columns d0+4q.. of row k0+e, and lane j receives column d0+j of rows
//     k0..k0+3, i.e. four consecutive keys of its own column, which is the key-contiguous operand
//     the MFMA needs. Two such reads form the 8-element operand.
// gfx950's LDS has 64 banks of 4 bytes, so a b128 read is served 16 lanes (256 bytes) and a b64
// read 32 lanes (256 bytes) at a time. The swizzle keeps both access patterns conflict-free: the 16
// lanes of a row read hit 16 distinct rows at one logical chunk, and the 32 lanes of a transpose
// read hit 4 consecutive rows x 4 consecutive chunks.
//
// Reference: pallas_attn.py:112-141 (forward), 161-215 (dQ, dK/dV), 274-311 (VJP driver).
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
template <int D>
struct TileDma {
  static constexpr int C = Tile<D>::C;
  static constexpr int RPO = Tile<D>::ROWS_PER_OP;
  uint32_t voff;

  __device__ __forceinline__ void init(int w, int lane, uint32_t snb) {
    const int row = w * RPO + lane / C;
    voff = (uint32_t)row * snb + (uint32_t)((((lane % C) ^ swz<C>(row))) << 4);
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

// ------------------------------------------------------------------------------------------
// Forward: per work item (a run of a query block's live tiles), O^T += V^T P^T with an online
// softmax (pallas_attn.py:112-141).
//
// Two workgroups per CU: one K buffer and one V buffer (64 KB at D = 128) and at most 256 VGPRs
// per wave, so the two resident workgroups overlap one's softmax (VALU) with the other's MFMAs.
// K(t+1) streams in during softmax(t) and PV(t), V(t+1) during S(t+1).
template <int D>
__global__ void __launch_bounds__(NT, 2) fwd_kernel(KArgs a) {
  constexpr int TB = Tile<D>::BYTES;
  __shared__ __attribute__((aligned(1024))) char lk[TB];
  __shared__ __attribute__((aligned(1024))) char lv[TB];
  lds_char* K = (lds_char*)lk;
  lds_char* V = (lds_char*)lv;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i = lane & 31, g = lane >> 5;
  const Job j = decode_job(a);
  const uint32_t snb = (uint32_t)a.sn * 2;
  const rsrc_t rK = make_rsrc((const uint16_t*)a.k + j.base, a.slice_bytes);
  const rsrc_t rV = make_rsrc((const uint16_t*)a.v + j.base, a.slice_bytes);

  const int qrow = j.blk * BLK + 32 * w + i;
  u32x4 qf[D / 16];
  load_frag<D>(qf, make_rsrc((const uint16_t*)a.q + j.base, a.slice_bytes), qrow, snb, g);
  Off<D> off;
  off.init(lane);
  TileDma<D> dma;
  dma.init(w, lane, snb);
  f32x16 o[D / 32];
#pragma unroll
  for (int db = 0; db < D / 32; ++db) o[db] = zero16();
  SoftmaxState st{-__builtin_inff(), 0.f};

  int t0, t1;
  tile_range(a, j, t0, t1);
  u32x2 mbits = {0u, 0u};  // mask bits of the next tile, loaded a tile ahead
  uint32_t gnext = 0u;     // group bits of the next tile, loaded a tile ahead
  if (t0 < t1) {
    const int kb = ((ci32_ptr)a.col)[t0];
    mbits = tile_bits(a, t0, w, lane);
    gnext = tile_groups(a, t0);
    dma.issue(rK, K, w, kb * BLK, snb);
    wait_vmem();  // K(t0), its mask and group bits and the Q fragment
    dma.issue(rV, V, w, kb * BLK, snb);
  }
  __syncthreads();
  for (int tt = t0; tt < t1; ++tt) {
    const int t = __builtin_amdgcn_readfirstlane(tt);
    // K(t) is in LDS for every wave here; V(t) may still be in flight.
    const u32x2 mb = mbits;
    const uint32_t gt = gnext;
    if (t + 1 < t1) {
      mbits = tile_bits(a, t + 1, w, lane);
      gnext = tile_groups(a, t + 1);
    }
    // Key groups with no valid element for this wave are skipped: they would add p = 0. Key
    // groups with none for any wave are not copied either.
    const uint32_t live = gt >> (4 * w) & 15u;
    const uint32_t full = gt >> (16 + 4 * w) & 15u;  // groups with every element valid: no mask
    f32x16 s[4];
    // MFMAs of every live group first, then the masks: a group's mask VALU work then waits on
    // MFMAs issued several groups earlier rather than on its own.
#pragma unroll
    for (int sb = 0; sb < 4; ++sb) {
      if (!(live >> sb & 1u)) continue;
      u32x4 ka[D / 16];
#pragma unroll
      for (int k = 0; k < D / 16; ++k) ka[k] = row_read(K, off.row[k] + sb * 32 * (2 * D));
      s[sb] = zero16();
#pragma unroll
      for (int k = 0; k < D / 16; ++k) s[sb] = mfma_bf16(ka[k], qf[k], s[sb]);
    }
#pragma unroll
    for (int sb = 0; sb < 4; ++sb) {
      if (!(live >> sb & 1u) || (full >> sb & 1u)) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) s[sb][r] = keep_or_ninf(s[sb][r], elem_keep(mb, sb, r));
    }
    wait_vmem();      // this wave's part of V(t); the next tile's group bits
    __syncthreads();  // all of V(t) landed; every wave is done reading K(t)
    const uint32_t copy_next = any_rows(gnext);
    if (t + 1 < t1) dma.issue(rK, K, w, ((ci32_ptr)a.col)[t + 1] * BLK, snb, copy_next);
    float corr;
    // The row max and the lazy rescale first; then per group the exponentials and its PV MFMAs,
    // so one group's VALU work overlaps the previous group's MFMAs.
    if (live != 0u && softmax_rebase(s, live, st, a.c2, corr)) {
#pragma unroll
      for (int db = 0; db < D / 32; ++db) o[db] *= corr;
    }
    const float base = softmax_base(st);
    float sum = 0.f;
#pragma unroll
    for (int sb = 0; sb < 4; ++sb) {
      if (!(live >> sb & 1u)) continue;
      u32x4 va[D / 32][2];
#pragma unroll
      for (int db = 0; db < D / 32; ++db)
#pragma unroll
        for (int c = 0; c < 2; ++c) va[db][c] = tr_operand<D>(V, off, db, sb, c);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = fast_exp2(fmaf(s[sb][r], a.c2, -base));
        s[sb][r] = p;
        sum += p;
      }
      const bf16x8 p0 = pack_bf16(s[sb], 0), p1 = pack_bf16(s[sb], 1);
#pragma unroll
      for (int db = 0; db < D / 32; ++db) {
        o[db] = mfma_bf16(va[db][0], p0, o[db]);
        o[db] = mfma_bf16(va[db][1], p1, o[db]);
      }
    }
    st.l += sum;
    wait_vmem();      // this wave's part of K(t+1)
    __syncthreads();  // all of K(t+1) landed; every wave is done reading V(t)
    if (t + 1 < t1) dma.issue(rV, V, w, ((ci32_ptr)a.col)[t + 1] * BLK, snb, copy_next);
  }
  const float ltot = st.l + __shfl_xor(st.l, 32);
  if (j.part >= 0) {
    store_fwd_partial<D>(a, j, 32 * w + i, o, st.m, ltot, g);
    return;
  }
  const float inv = ltot > 0.f ? 1.f / ltot : 0.f;
  store_acc_bf16<D>(make_rsrc((uint16_t*)a.out0 + j.obase, a.oslice_bytes), qrow, (uint32_t)a.osn * 2, o, inv, g);
  if (g == 0) write_lse(a, j, qrow, st, ltot);
}

// ------------------------------------------------------------------------------------------
// dQ: per work item of the forward tile list (pallas_attn.py:161-184).
// P = where(valid, exp(s*scale - lse), 0); dS = P * (dP - delta); dQ = scale * dS K.
//
// Two workgroups per CU: single K and V buffers (64 KB at D = 128), refilled once every wave is
// done with the tile, and at most 256 VGPRs per wave; the other resident workgroup computes while
// the copy is in flight.
template <int D>
__global__ void __launch_bounds__(NT, 2) dq_kernel(KArgs a) {
  constexpr int TB = Tile<D>::BYTES;
  __shared__ __attribute__((aligned(1024))) char lk[TB];
  __shared__ __attribute__((aligned(1024))) char lv[TB];
  lds_char* K = (lds_char*)lk;
  lds_char* V = (lds_char*)lv;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i = lane & 31, g = lane >> 5;
  const Job j = decode_job(a);
  const uint32_t snb = (uint32_t)a.sn * 2;
  const rsrc_t rK = make_rsrc((const uint16_t*)a.k + j.base, a.slice_bytes);
  const rsrc_t rV = make_rsrc((const uint16_t*)a.v + j.base, a.slice_bytes);

  const int qrow = j.blk * BLK + 32 * w + i;
  u32x4 qf[D / 16], df[D / 16];
  load_frag<D>(qf, make_rsrc((const uint16_t*)a.q + j.base, a.slice_bytes), qrow, snb, g);
  load_frag<D>(df, make_rsrc((const uint16_t*)a.dout + j.obase, a.oslice_bytes), qrow, (uint32_t)a.osn * 2, g);
  float lse_t = 0.f, delta = 0.f;
  if (qrow < a.n) {
    lse_t = a.lse[stat_index(a, j, qrow)] * LOG2E;
    delta = a.delta[stat_index(a, j, qrow)];
  }
  Off<D> off;
  off.init(lane);
  TileDma<D> dma;
  dma.init(w, lane, snb);
  f32x16 acc[D / 32];
#pragma unroll
  for (int db = 0; db < D / 32; ++db) acc[db] = zero16();

  int t0, t1;
  tile_range(a, j, t0, t1);
  // Each tile is copied in two halves: rows 0-63 (key groups 0-1) and rows 64-127 (groups 2-3).
  // A half of tile t+1 is copied while the other half of tile t is computed, so every copy has
  // half a tile of work to hide behind. Per tile: wait + barrier, copy the second half of t,
  // groups 0-1 of t, wait + barrier, copy the first half of t+1, groups 2-3 of t.
  u32x2 mbits = {0u, 0u};  // mask bits of the next tile, loaded with its first half
  uint32_t gcur = 0u, gnext = 0u, hcur = 0u, hnext = 0u;
  if (t0 < t1) {
    const int kb = ((ci32_ptr)a.col)[t0];
    mbits = tile_bits(a, t0, w, lane);
    gcur = tile_groups(a, t0);
    hcur = tile_halves(a, t0);
    dma.issue(rK, K, w, kb * BLK, snb, 3u);
    dma.issue(rV, V, w, kb * BLK, snb, 3u);
  }
  // hv: this wave's live 16-key halves of the group (bit h); a clear half gets no dS work and
  // no dQ MFMAs (its dS is zero).
  auto group = [&](int sb, const u32x2& mb, bool full, uint32_t hv) {
    u32x4 ka[D / 16], va[D / 16];
#pragma unroll
    for (int k = 0; k < D / 16; ++k) {
      ka[k] = row_read(K, off.row[k] + sb * 32 * (2 * D));
      va[k] = row_read(V, off.row[k] + sb * 32 * (2 * D));
    }
    __builtin_amdgcn_sched_barrier(0);
    f32x16 s = zero16(), dp = zero16();
#pragma unroll
    for (int k = 0; k < D / 16; ++k) {
      s = mfma_bf16(ka[k], qf[k], s);
      dp = mfma_bf16(va[k], df[k], dp);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      if (!(hv >> h & 1u)) continue;
      u32x4 kt[D / 32];
#pragma unroll
      for (int db = 0; db < D / 32; ++db) kt[db] = tr_operand<D>(K, off, db, sb, h);
      __builtin_amdgcn_sched_barrier(0);
      if (full) {  // every element of the group is valid
#pragma unroll
        for (int r = 8 * h; r < 8 * h + 8; ++r) dp[r] = fast_exp2(fmaf(s[r], a.c2, -lse_t)) * (dp[r] - delta);
      } else {
#pragma unroll
        for (int r = 8 * h; r < 8 * h + 8; ++r) {
          const float p = keep_or_zero(fast_exp2(fmaf(s[r], a.c2, -lse_t)), elem_keep(mb, sb, r));
          dp[r] = p * (dp[r] - delta);
        }
      }
      const bf16x8 dh = pack_bf16(dp, h);
#pragma unroll
      for (int db = 0; db < D / 32; ++db) acc[db] = mfma_bf16(kt[db], dh, acc[db]);
    }
  };
  for (int tt = t0; tt < t1; ++tt) {
    const int t = __builtin_amdgcn_readfirstlane(tt);
    const int kb = ((ci32_ptr)a.col)[t];
    wait_vmem();      // this wave's part of rows 0-63 of tile t and its mask bits
    __syncthreads();  // all of rows 0-63 landed; every wave is done with rows 64-127 of tile t-1
    const u32x2 mb = mbits;
    const uint32_t gt = gcur;
    const uint32_t hw = hcur >> (8 * w) & 0xffu;  // this wave's live halves: bit 2sb + h
    if (t + 1 < t1) {
      gnext = tile_groups(a, t + 1);
      hnext = tile_halves(a, t + 1);
    }
    const uint32_t copy = any_rows(gt);
    dma.issue(rK, K, w, kb * BLK, snb, copy & 12u);
    dma.issue(rV, V, w, kb * BLK, snb, copy & 12u);
    // Key groups with no valid element for this wave are skipped (p = 0 throughout); key groups
    // with none for any wave are not copied either.
    const uint32_t live = gt >> (4 * w) & 15u;
    const uint32_t full = gt >> (16 + 4 * w) & 15u;  // groups with every element valid: no mask
    if (live & 1u) group(0, mb, full & 1u, hw & 3u);
    if (live & 2u) group(1, mb, full & 2u, hw >> 2 & 3u);
    wait_vmem();      // this wave's part of rows 64-127 of tile t
    __syncthreads();  // all of rows 64-127 landed; every wave is done with rows 0-63 of tile t
    if (t + 1 < t1) {
      const int kb1 = ((ci32_ptr)a.col)[t + 1];
      const uint32_t copy1 = any_rows(gnext);
      mbits = tile_bits(a, t + 1, w, lane);
      dma.issue(rK, K, w, kb1 * BLK, snb, copy1 & 3u);
      dma.issue(rV, V, w, kb1 * BLK, snb, copy1 & 3u);
    }
    if (live & 4u) group(2, mb, full & 4u, hw >> 4 & 3u);
    if (live & 8u) group(3, mb, full & 8u, hw >> 6 & 3u);
    gcur = gnext;
    hcur = hnext;
  }
  if (j.part >= 0) {
    store_bwd_partial<D>(a, j, 32 * w + i, acc, 0, g);
    return;
  }
  store_acc_bf16<D>(make_rsrc((uint16_t*)a.out0 + j.base, a.slice_bytes), qrow, snb, acc, a.scale, g);
}

// ------------------------------------------------------------------------------------------
// dK/dV: per work item of the transposed tile list; each workgroup owns its dK/dV rows, so there
// are no atomics (pallas_attn.py:187-215). The tile's 128 log-sum-exps and deltas are copied next
// to its Q and dO tiles; the log-sum-exps are rescaled to the log2 domain once per tile in LDS.
//
// The work is split by role over 8 waves. Waves w and w + 4 share one SIMD and own the same 32
// keys. Wave w (the P wave) holds the K fragment and computes S^T = K Q^T and P, hands P over
// to wave w + 4 through LDS and accumulates the first half of dV's columns. Wave w + 4 holds the
// V fragment and computes dP^T = V dO^T, dS = P (dP - delta), dK += dS^T Q and the second half
// of dV's columns (all of them at D = 32). Splitting dV moves MFMAs off the P wave, whose
// exponentials otherwise keep the other wave waiting at every hand-over.
constexpr int NT8 = 512;
constexpr int PSLOT = 2048;  // one P slot: 32 keys x 32 queries bf16

template <int D>
__global__ void __launch_bounds__(NT8, 1) dkv_kernel(KArgs a) {
  constexpr int TB = Tile<D>::BYTES;
  constexpr int NB = D / 32;     // 32-column blocks of dK and dV
  constexpr int NV0 = NB / 2;    // dV blocks of the P wave (none at D = 32)
  constexpr int NV1 = NB - NV0;  // dV blocks of the dK wave
  __shared__ __attribute__((aligned(1024))) char lds0[2 * TB + 1536];  // Q | dO | lse[128] | gap | delta[128]
  __shared__ __attribute__((aligned(1024))) char lds1[2 * TB + 1536];
  __shared__ __attribute__((aligned(1024))) char lp[4 * 2 * PSLOT];  // 2 P slots per key sub-block
  lds_char* bufs[2] = {(lds_char*)lds0, (lds_char*)lds1};
  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int w = wid & 3;        // key sub-block
  const bool kw = wid >= 4;     // dK wave (else P wave)
  const int i = lane & 31, g = lane >> 5;
  const Job j = decode_job(a);
  const uint32_t snb = (uint32_t)a.sn * 2;
  const rsrc_t rQ = make_rsrc((const uint16_t*)a.q + j.base, a.slice_bytes);
  const rsrc_t rO = make_rsrc((const uint16_t*)a.dout + j.obase, a.oslice_bytes);
  const uint32_t osnb = (uint32_t)a.osn * 2;
  const rsrc_t rL = make_rsrc(a.lse + stat_index(a, j, 0), (uint32_t)a.n * 4);
  const rsrc_t rD = make_rsrc(a.delta + stat_index(a, j, 0), (uint32_t)a.n * 4);

  const int krow = j.blk * BLK + 32 * w + i;  // this lane's key
  u32x4 frag[D / 16];                          // K (P waves) or V (dK waves)
  load_frag<D>(frag, make_rsrc((const uint16_t*)(kw ? a.v : a.k) + j.base, a.slice_bytes), krow, snb, g);
  Off<D> off;
  off.init(lane);
  TileDma<D> dma, dmaO;  // Q and dO tiles (their row strides may differ)
  dma.init(w, lane, snb);
  dmaO.init(w, lane, osnb);
  f32x16 acc[NB];    // dK (dK waves) or dV blocks 0 .. NV0 - 1 (P waves)
  f32x16 accv[NV1];  // dV blocks NV0 .. NB - 1 (dK waves)
#pragma unroll
  for (int db = 0; db < NB; ++db) acc[db] = zero16();
#pragma unroll
  for (int db = 0; db < NV1; ++db) accv[db] = zero16();
  // A P slot holds the two 8-element halves of every lane, each half 64 lanes x 16 bytes
  // contiguous, so the slot's b128 writes and reads are free of bank conflicts.
  lds_char* pslot = (lds_char*)lp + w * 2 * PSLOT + lane * 16;

  int t0, t1;
  tile_range(a, j, t0, t1);
  constexpr uint32_t kPastEnd = 0x7FFFFFF0u;
  // The P waves copy the tiles, their statistics and their mask bits.
  auto issue = [&](int t, lds_char* buf, uint32_t copy) {
    const int qb = ((ci32_ptr)a.col)[t];
    dma.issue(rQ, buf, w, qb * BLK, snb, copy);
    dmaO.issue(rO, buf + TB, w, qb * BLK, osnb, copy);
    if (wid == 0) {
      const uint32_t vo = (uint32_t)(qb * BLK + 4 * (lane & 31)) * 4;
      lds_char* stats = buf + 2 * TB;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rL, (__attribute__((address_space(3))) void*)stats, 16,
                                               (int)(lane < 32 ? vo : kPastEnd), 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rD, (__attribute__((address_space(3))) void*)(stats + 512), 16,
                                               (int)(lane < 32 ? kPastEnd : vo), 0, 0, 0);
    }
  };
  auto stats4 = [&](const lds_char* cur, int off_bytes, int sb, f32x4 (&x)[4]) {
    const __attribute__((address_space(3))) float* p =
        (const __attribute__((address_space(3))) float*)(cur + 2 * TB + off_bytes);
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
        x[2 * c + hh] = *(const __attribute__((address_space(3))) f32x4*)(p + 32 * sb + 16 * c + 8 * g + 4 * hh);
  };
  // Query groups (32 queries) of a tile with no valid element for any of the 4 key groups are
  // skipped by every wave and not copied (they would add p = 0); the others cost one barrier each,
  // so per tile each wave passes 1 + (number of live query groups) barriers. A dK wave also skips
  // the live groups in which its own 32 keys have no valid element (its P is zero there). The P
  // waves compute every live group: the barriers pace all 8 waves, so a skip there would only
  // move the wait to another wave. Group bits are loaded a tile ahead of their use (two tiles
  // ahead of the copy for P waves).
  u32x2 mbits = {0u, 0u};
  uint32_t gcur = 0u, gnext = 0u;  // group bits of the current and (P waves) the next tile
  if (t0 < t1) gcur = tile_groups(a, t0);
  if (t0 < t1 && !kw) {
    mbits = tile_bits(a, t0, w, lane);
    if (t0 + 1 < t1) gnext = tile_groups(a, t0 + 1);
    issue(t0, bufs[0], 15u);
  }
  auto pv_step = [&](int tt, lds_char* cur, lds_char* nxt) {
    const int t = __builtin_amdgcn_readfirstlane(tt);
    wait_vmem();
    const u32x2 mb = mbits;
    if (wid == 0) {
      // lse -> -lse / scale and delta -> -delta, the initial values of the S^T and dP^T
      // accumulators: (s - lse / scale) * c2 = s * c2 - lse * log2(e), and dP - delta.
      __attribute__((address_space(3))) f32x4* x =
          (__attribute__((address_space(3))) f32x4*)(cur + 2 * TB + (lane < 32 ? 0 : 512) + 16 * lane);
      float m = lane < 32 ? a.nlse_mul : -1.f;
      asm volatile("" : "+v"(m));  // computed here: hoisted, the compiler keeps it as spilled vectors
      *x = *x * m;
    }
    __syncthreads();  // tile t is in LDS; every wave is done with tile t - 1 (buffer nxt)
    const uint32_t any = any_rows(gcur);
    if (t + 1 < t1) {
      mbits = tile_bits(a, t + 1, w, lane);
      issue(t + 1, nxt, any_rows(gnext));
    }
    gcur = gnext;
    if (t + 2 < t1) gnext = tile_groups(a, t + 2);
    const lds_char* Q = cur;
    const lds_char* O = cur + TB;
    // S^T of query group sb, started at -lse / scale of the element's query.
    auto s_chain = [&](int sb) {
      u32x4 qa[D / 16];
#pragma unroll
      for (int k = 0; k < D / 16; ++k) qa[k] = row_read(Q, off.row[k] + sb * 32 * (2 * D));
      f32x4 lr[4];
      stats4(cur, 0, sb, lr);
      f32x16 sv;
#pragma unroll
      for (int r = 0; r < 16; ++r) sv[r] = lr[r >> 2][r & 3];
#pragma unroll
      for (int k = 0; k < D / 16; ++k) sv = mfma_bf16(qa[k], frag[k], sv);
      return sv;
    };
    // P = exp2(S c2) (masked), packed to bf16 and written to LDS slot `slot` for the dK wave.
    auto finish_p = [&](f32x16& sv, int sb, int slot, bf16x8& p0, bf16x8& p1) {
#pragma unroll
      for (int r = 0; r < 16; ++r) sv[r] = keep_or_zero(fast_exp2(sv[r] * a.c2), elem_keep(mb, sb, r));
      p0 = pack_bf16(sv, 0);
      p1 = pack_bf16(sv, 1);
      lds_char* ps = pslot + slot * PSLOT;
      *(__attribute__((address_space(3))) bf16x8*)ps = p0;
      *(__attribute__((address_space(3))) bf16x8*)(ps + 1024) = p1;
    };
    // P runs one live query group ahead. Between two barriers this wave computes S(next), then
    // issues its dV(sb) MFMAs one at a time between slices of next's exponentials, so that the
    // VALU work runs while the MFMA pipe is busy; the dK wave meanwhile issues dK(sb), its dV(sb)
    // and dP(next). P(sb) goes to slot (its rank in `any`) & 1.
    bf16x8 pc0, pc1;
    if (any != 0u) {
      const int sb0 = __builtin_ctz(any);
      f32x16 sv = s_chain(sb0);
      finish_p(sv, sb0, 0, pc0, pc1);
    }
    int rank = 0;
#pragma unroll
    for (int sb = 0; sb < 4; ++sb) {
      if (!(any >> sb & 1u)) continue;
      lds_barrier();  // P(sb) is in LDS for the dK wave
      ++rank;
      const uint32_t later = sb < 3 ? any & (0xeu << sb) : 0u;
      u32x4 ot[NV0 > 0 ? NV0 : 1][2];
      if (later != 0u) {
        const int nsb = __builtin_ctz(later);
        f32x16 sv = s_chain(nsb);
#pragma unroll
        for (int db = 0; db < NV0; ++db)
#pragma unroll
          for (int c = 0; c < 2; ++c) ot[db][c] = tr_operand<D>(O, off, db, sb, c);
        // Order: the Q and stats reads; the S chain with the dO^T reads between its MFMAs
        // (they take the registers the Q operands free); then the dV MFMAs with slices of the
        // exponential work between them; the P slot writes.
        __builtin_amdgcn_sched_group_barrier(0x100, D / 16 + 4, 0);
#pragma unroll
        for (int m = 0; m < D / 16; ++m) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          if (m < 4 * NV0) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        bf16x8 pn0, pn1;
#pragma unroll
        for (int db = 0; db < NV0; ++db) {
          acc[db] = mfma_bf16(ot[db][0], pc0, acc[db]);
          acc[db] = mfma_bf16(ot[db][1], pc1, acc[db]);
        }
        finish_p(sv, nsb, rank & 1, pn0, pn1);
        if constexpr (NV0 > 0) {
#pragma unroll
          for (int m = 0; m < 2 * NV0; ++m) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
            __builtin_amdgcn_sched_group_barrier(0x002, 80 / (2 * NV0), 1);
          }
          __builtin_amdgcn_sched_group_barrier(0x200, 2, 1);
        }
        pc0 = pn0;
        pc1 = pn1;
      } else {
#pragma unroll
        for (int db = 0; db < NV0; ++db)
#pragma unroll
          for (int c = 0; c < 2; ++c) ot[db][c] = tr_operand<D>(O, off, db, sb, c);
#pragma unroll
        for (int db = 0; db < NV0; ++db) {
          acc[db] = mfma_bf16(ot[db][0], pc0, acc[db]);
          acc[db] = mfma_bf16(ot[db][1], pc1, acc[db]);
        }
      }
    }
  };
  auto dk_step = [&](int tt, lds_char* cur) {
    __syncthreads();
    const uint32_t any = any_rows(gcur), own = gcur >> (4 * w) & 15u;
    if (tt + 1 < t1) gcur = tile_groups(a, tt + 1);
    const lds_char* Q = cur;
    const lds_char* O = cur + TB;
    int rank = 0;
#pragma unroll
    for (int sb = 0; sb < 4; ++sb) {
      if (!(any >> sb & 1u)) continue;
      const bool mine = own >> sb & 1u;
      f32x16 dp;
      u32x4 qt[NB][2];
      if (mine) {
        u32x4 oa[D / 16];
#pragma unroll
        for (int k = 0; k < D / 16; ++k) oa[k] = row_read(O, off.row[k] + sb * 32 * (2 * D));
        f32x4 dr[4];
        stats4(cur, 1024, sb, dr);
#pragma unroll
        for (int r = 0; r < 16; ++r) dp[r] = dr[r >> 2][r & 3];  // -delta of the element's query
#pragma unroll
        for (int k = 0; k < D / 16; ++k) dp = mfma_bf16(oa[k], frag[k], dp);
#pragma unroll
        for (int db = 0; db < NB; ++db)
#pragma unroll
          for (int c = 0; c < 2; ++c) qt[db][c] = tr_operand<D>(Q, off, db, sb, c);
      }
      lds_barrier();  // P(sb) written by the P wave
      if (mine) {
        const lds_char* ps = pslot + (rank & 1) * PSLOT;
        const u32x4 pw0 = *(const __attribute__((address_space(3))) u32x4*)ps;
        const u32x4 pw1 = *(const __attribute__((address_space(3))) u32x4*)(ps + 1024);
        u32x4 ot[NV1][2];
#pragma unroll
        for (int db = 0; db < NV1; ++db)
#pragma unroll
          for (int c = 0; c < 2; ++c) ot[db][c] = tr_operand<D>(O, off, NV0 + db, sb, c);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const uint32_t word = (r < 8 ? pw0 : pw1)[(r & 7) >> 1];
          const float p = __builtin_bit_cast(float, (r & 1) ? (word & 0xffff0000u) : (word << 16));
          dp[r] = p * dp[r];
        }
        const bf16x8 d0 = pack_bf16(dp, 0), d1 = pack_bf16(dp, 1);
#pragma unroll
        for (int db = 0; db < NB; ++db) {
          acc[db] = mfma_bf16(qt[db][0], d0, acc[db]);
          acc[db] = mfma_bf16(qt[db][1], d1, acc[db]);
        }
        const bf16x8 p0 = __builtin_bit_cast(bf16x8, pw0), p1 = __builtin_bit_cast(bf16x8, pw1);
#pragma unroll
        for (int db = 0; db < NV1; ++db) {
          accv[db] = mfma_bf16(ot[db][0], p0, accv[db]);
          accv[db] = mfma_bf16(ot[db][1], p1, accv[db]);
        }
      }
      ++rank;
    }
  };
  if (!kw) {
    for (int tt = t0; tt < t1; tt += 2) {
      pv_step(tt, bufs[0], bufs[1]);
      if (tt + 1 < t1) pv_step(tt + 1, bufs[1], bufs[0]);
    }
  } else {
    for (int tt = t0; tt < t1; tt += 2) {
      dk_step(tt, bufs[0]);
      if (tt + 1 < t1) dk_step(tt + 1, bufs[1]);
    }
  }
  const rsrc_t rV = make_rsrc((uint16_t*)a.out1 + j.base, a.slice_bytes);
  if (kw) {
    if (j.part >= 0) {
      store_bwd_partial<D>(a, j, 32 * w + i, acc, 0, g);
      store_bwd_partial<D, NV1>(a, j, 32 * w + i, accv, 1, g, NV0);
      return;
    }
    store_acc_bf16<D>(make_rsrc((uint16_t*)a.out0 + j.base, a.slice_bytes), krow, snb, acc, a.scale, g);
    store_acc_bf16<D, NV1>(rV, krow, snb, accv, 1.f, g, NV0);
  } else if constexpr (NV0 > 0) {
    f32x16 dv[NV0];
#pragma unroll
    for (int db = 0; db < NV0; ++db) dv[db] = acc[db];
    if (j.part >= 0) {
      store_bwd_partial<D, NV0>(a, j, 32 * w + i, dv, 1, g, 0);
      return;
    }
    store_acc_bf16<D, NV0>(rV, krow, snb, dv, 1.f, g, 0);
  }
}

template <int D>
hipError_t launch_d(Kind kind, const KArgs& a, hipStream_t stream) {
  const dim3 grid((unsigned)a.n_items * (unsigned)(a.batch * a.heads)), block(NT);
  switch (kind) {
    case Kind::kFwd: hipLaunchKernelGGL(fwd_kernel<D>, grid, block, 0, stream, a); break;
    case Kind::kDq: hipLaunchKernelGGL(dq_kernel<D>, grid, block, 0, stream, a); break;
    case Kind::kDkv: hipLaunchKernelGGL(dkv_kernel<D>, grid, dim3(NT8), 0, stream, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_bf16(Kind kind, int head_dim, const KArgs& a, hipStream_t stream) {
  switch (head_dim) {
    case 32: return launch_d<32>(kind, a, stream);
    case 64: return launch_d<64>(kind, a, stream);
    case 128: return launch_d<128>(kind, a, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace fwn
