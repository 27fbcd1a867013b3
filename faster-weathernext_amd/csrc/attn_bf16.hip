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
// gfx950's LDS has 64 banks of 4 bytes. A b128 read is served 16 lanes (256 bytes) at a time
// (measured: the lanes of one half-wave whose quad index l / 4 has the same parity), a b64
// transpose read 32 lanes (256 bytes). The swizzle keeps both access patterns conflict-free
// (measured: no conflict cycles in the forward): the lanes of a row read hit distinct rows at one
// logical chunk, and the 32 lanes of a transpose read hit 4 consecutive rows x 4 consecutive
// chunks.
//
// Reference: pallas_attn.py:112-141 (forward), 161-215 (dQ, dK/dV), 274-311 (VJP driver).
#include "attn_bf16_tiles.h"

namespace fwn {
namespace {

using namespace dev;

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
  if (j.skip) return;  // an empty entry of the order table
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
      // All of the group's K reads are issued before its MFMA chain: the chain then waits for
      // the LDS latency once, not once per pair of MFMAs.
      __builtin_amdgcn_sched_barrier(0);
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
      // The V transpose reads are all in flight while the exponentials run.
      __builtin_amdgcn_sched_barrier(0);
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
  if (j.skip) return;  // an empty entry of the order table
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
// The dS exchange (bf16 backward): dkv16_kernel<D, true> writes every 32 x 16 unit of dS it
// computes, dq_ds_kernel reads it instead of recomputing S and dP.
//
// A unit is one dK/dV wave's 16 keys x one 32-query group of a tile, which is exactly the 16-key
// half (key group kg / 2, half kg % 2) of one dQ wave's 32 query rows. dK/dV stores it as its
// registers hold it, 1 KB, 16 bytes per lane: lane L' = k + 16 g writes the bf16 dS of key k for
// queries 4g..4g+3, then 16+4g..16+4g+3. The dQ contraction runs over keys, so its B operand
// (V_MFMA_F32_32X32X16_BF16, lane L: query L % 32, keys 8 (L / 32) .. +7) is the transpose; the
// dQ kernel does that transpose through LDS, where it has bandwidth to spare (dK/dV has none).
// Lane L writes chunk L to 16-byte slot p(k, g) = 16 (k / 4) + 4 (g ^ (k / 4)) + k % 4, then two
// transpose reads (ds_read_b64_tr_b16: lane j of a 16-lane group gets column d0 + j of 4 rows)
// give keys 8 (L / 32) .. +3 and +4 .. +7 of query L % 32.
// LDS service on gfx950, measured with single-pattern probes (SQ_LDS_BANK_CONFLICT): a
// ds_write_b128 is served 8 consecutive lanes per cycle, without conflict when their 16-byte
// chunks are distinct modulo 128 bytes; here lanes 8m .. 8m + 7 (keys 8 (m % 2) .. +7, one g) write
// p mod 8 = 4 ((g ^ (k / 4)) % 2) + k % 4, eight distinct values. The transpose reads hit 32
// distinct bank pairs over lanes 0-31 and over lanes 32-63 (keys k0 .. k0 + 3 of one quarter:
// 4 (q ^ (k / 4)) + k % 4 takes 16 values, times the two halves). An earlier slot order,
// 16 (k / 4) + 4 (k % 4) + (g ^ (k / 4)), put keys k and k + 2 on one 128-byte position: every
// write group 2-way, 8 conflict cycles per unit, 22% of the kernel's LDS cycles.
constexpr int kNonTemporal = 2;  // buffer store cache policy: non-temporal (gfx950 "nt")

struct DsUnit {
  uint32_t w;       // this lane's write: byte offset of slot p(L % 16, L / 16)
  uint32_t r0, r1;  // this lane's transpose reads: keys 8 (L / 32) .. +3 and +4 .. +7

  static __device__ __forceinline__ uint32_t slot(int k, int g) {
    return (uint32_t)(16 * (16 * (k >> 2) + 4 * (g ^ (k >> 2)) + (k & 3)));
  }
  __device__ __forceinline__ void init(int lane) {
    w = slot(lane & 15, lane >> 4);
    const int gg = lane >> 4, e = (lane >> 2) & 3, q = lane & 3, k0 = 8 * (gg >> 1);
    r0 = slot(k0 + e, q) + 8u * (gg & 1);
    r1 = slot(k0 + 4 + e, q) + 8u * (gg & 1);
  }
};

// dQ from the dS units (pallas_attn.py:177-184, with dS taken from the dK/dV pass instead of
// recomputed): per work item of the forward list, dQ^T += K^T dS^T over the live 16-key halves of
// each wave's 32 query rows. Each live half is one unit, loaded with one 16-byte load per lane
// and transposed through this wave's LDS stage (DsUnit): no S, no dP, no exponentials, one of
// dq_kernel's three contractions.
//
// K tiles are double-buffered in LDS (64 KB at D = 128, one barrier per tile), two workgroups per
// CU. After the barrier of tile t the K rows of tile t + 1 are requested, and its dS units after
// the first half's LDS work, so both arrive while tile t is computed; the column block, half bits
// and first unit of tile t + 3 are read with scalar loads at the end of the step. Within a tile
// the wave's live halves run as a two-stage pipeline: half k + 1's unit goes through the other
// 1 KB stage slot and its LDS reads are in flight while half k's MFMAs issue (C3 dQ -2% against
// one key group at a time, whose MFMAs waited for all of the group's reads).
template <int D>
__global__ void __launch_bounds__(NT, 2) dq_ds_kernel(KArgs a) {
  constexpr int TB = Tile<D>::BYTES;
  __shared__ __attribute__((aligned(1024))) char lk0[TB];
  __shared__ __attribute__((aligned(1024))) char lk1[TB];
  __shared__ __attribute__((aligned(1024))) char lstage[4 * 2048];  // per wave: two unit slots
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i = lane & 31, g = lane >> 5;
  const Job j = decode_job(a);
  if (j.skip) return;  // an empty entry of the order table
  const uint32_t snb = (uint32_t)a.sn * 2;
  const rsrc_t rK = make_rsrc((const uint16_t*)a.k + j.base, a.slice_bytes);
  const rsrc_t rS = make_rsrc(a.ds + (int64_t)j.bh * (a.ds_slice_bytes >> 1), a.ds_slice_bytes);
  lds_char* st = (lds_char*)lstage + 2048 * w;
  DsUnit du;
  du.init(lane);
  const int qrow = j.blk * BLK + 32 * w + i;
  Off<D> off;
  off.init(lane);
  TileDma<D> dma;
  dma.init(w, lane, snb);
  f32x16 acc[D / 32];
#pragma unroll
  for (int db = 0; db < D / 32; ++db) acc[db] = zero16();
  typedef const __attribute__((address_space(4))) int32_t* cmap_ptr;

  // This wave's units of a tile, in the order of its set half bits 8w .. 8w + 7: a tile's units
  // are numbered by rank among all of the word's set bits, so the wave's are consecutive, from
  // the tile's first unit plus the set bits of the waves before it. Each unit is read once:
  // non-temporal loads. The unit's offset is part of the per-lane offset, which the buffer unit
  // checks against the slice size (the scalar offset is not checked), so a dS map that does not
  // match the list cannot reach past its slice.
  auto load_units = [&](u32x4 (&dst)[8], uint32_t hf, uint32_t ub) {
    const uint32_t n = (uint32_t)__builtin_popcount(hf >> (8 * w) & 0xffu);
    const uint32_t u0 = ub + (uint32_t)__builtin_popcount(hf & ((1u << (8 * w)) - 1u));
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if ((uint32_t)k < n)
        dst[k] = __builtin_amdgcn_raw_buffer_load_b128(rS, (int)(16u * lane + (u0 + (uint32_t)k) * 1024u), 0, kNonTemporal);
  };
  // One live half: its unit through stage slot k % 2 (the slot's previous reads come first in
  // program order, and LDS runs one wave's accesses in order), then the dS^T operand and the
  // half's K^T operands (keys 16x .. 16x + 15, x = 2 sb + h the half's bit) into set `o`.
  struct HalfOps {
    u32x4 kt[D / 32], bs;
  };
  auto issue = [&](HalfOps& o, int k, const lds_char* K, uint32_t x, const u32x4& unit) {
    typedef __attribute__((address_space(3))) u32x4* l4p;
    *(l4p)(st + 1024 * (k & 1) + du.w) = unit;
    const u32x2 x0 = tr_read(st + 1024 * (k & 1), du.r0), x1 = tr_read(st + 1024 * (k & 1), du.r1);
    o.bs = u32x4{x0[0], x0[1], x1[0], x1[1]};
    const lds_char* Kx = K + x * (16u * 2u * D);
#pragma unroll
    for (int db = 0; db < D / 32; ++db) {
      const u32x2 lo = tr_read(Kx, off.tr[db][0]), hi = tr_read(Kx, off.tr[db][1]);
      o.kt[db] = u32x4{lo[0], lo[1], hi[0], hi[1]};
    }
  };
  auto mfmas = [&](const HalfOps& o) {
#pragma unroll
    for (int db = 0; db < D / 32; ++db) acc[db] = mfma_bf16(o.kt[db], o.bs, acc[db]);
  };

  // The tile copy at 16-row granularity: only the K rows of 16-key halves live in some wave are
  // read (live16 bit x: rows 16x .. 16x + 15), so the others are not copied (12% of the rows of
  // live 32-row groups at C3, 6% at the C5 shape; dQ -2% and -1.3%). Op `op` of this wave fills
  // rows 4 RPO op + RPO w .. + RPO - 1, inside one 16-row chunk.
  auto copy16 = [&](lds_char* tile, int row0, uint32_t live16) {
    constexpr int RPO = Tile<D>::ROWS_PER_OP;
    uint32_t base = (uint32_t)(uintptr_t)tile + (uint32_t)w * 1024u;
    asm volatile("" : "+s"(base));
#pragma unroll
    for (int op = 0; op < Tile<D>::OPS_PER_WAVE; ++op) {
      if (!(live16 >> ((op * 4 * RPO + w * RPO) >> 4) & 1u)) continue;
      const uint32_t vo = dma.voff + (uint32_t)(row0 + op * 4 * RPO) * snb;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rK, (__attribute__((address_space(3))) void*)(uintptr_t)(base + op * 4096u),
                                               16, (int)vo, 0, 0, 0);
    }
  };
  auto live16 = [](uint32_t hf) { return (hf | hf >> 8 | hf >> 16 | hf >> 24) & 0xffu; };

  int t0, t1;
  tile_range(a, j, t0, t1);
  // Scalars of tile t + 1 (c1, h1, u1: column block, half bits, first unit) and of tile t + 2
  // (c2, h2, u2), at the start of step t.
  int c1 = 0, c2 = 0;
  uint32_t h1 = 0u, h2 = 0u, u1 = 0u, u2 = 0u;
  u32x4 dsA[8], dsB[8];
  uint32_t hcur = 0u;
  // Step t: the live halves of tile t run as a two-stage pipeline, the LDS reads of half k + 1
  // in flight while the MFMAs of half k issue.
  auto step = [&](int tt, const lds_char* cur, lds_char* nxt, const u32x4 (&dsc)[8], u32x4 (&dsn)[8]) {
    const int t = __builtin_amdgcn_readfirstlane(tt);
    wait_vmem();      // this wave's part of tile t's K rows and its dS units
    __syncthreads();  // all of tile t's K rows landed; every wave is done with tile t - 1 (buffer nxt)
    const uint32_t ht = hcur;
    const bool more = t + 1 < t1;
    const uint32_t hl = h1, ul = u1;
    if (more) copy16(nxt, c1 * BLK, live16(h1));
    hcur = h1;
    c1 = c2;
    h1 = h2;
    u1 = u2;
    uint32_t rem = ht >> (8 * w) & 0xffu;
    const uint32_t n = (uint32_t)__builtin_popcount(rem);
    HalfOps P, Q;
    // Tile t + 1's units after the first half's LDS work: the K copy, which the next barrier
    // waits for, enters the buffer unit first (units first: C3 dQ +4%, C5 shape +6%; units right
    // after the copy: C5 shape +1.2% against this order).
    if (n != 0u) issue(P, 0, cur, (uint32_t)__builtin_ctz(rem), dsc[0]);
    if (more) load_units(dsn, hl, ul);
    if (n != 0u) {
      rem &= rem - 1u;
#pragma unroll
      for (int k = 1; k < 8; ++k) {
        if ((uint32_t)k < n) {
          if (k & 1) {
            issue(Q, k, cur, (uint32_t)__builtin_ctz(rem), dsc[k]);
            mfmas(P);
          } else {
            issue(P, k, cur, (uint32_t)__builtin_ctz(rem), dsc[k]);
            mfmas(Q);
          }
          rem &= rem - 1u;
        }
      }
      // The last live half's MFMAs: one call site, its operands selected by the half's parity (a
      // branch per set would give the accumulators two register assignments and copies between).
      const bool odd = ((n - 1u) & 1u) != 0u;
      HalfOps F;
      F.bs = odd ? Q.bs : P.bs;
#pragma unroll
      for (int db = 0; db < D / 32; ++db) F.kt[db] = odd ? Q.kt[db] : P.kt[db];
      mfmas(F);
    }
    if (t + 3 < t1) {
      c2 = ((ci32_ptr)a.col)[t + 3];
      h2 = tile_halves(a, t + 3);
      u2 = (uint32_t)((cmap_ptr)a.ubase)[t + 3];
    }
  };
  lds_char* K0 = (lds_char*)lk0;
  lds_char* K1 = (lds_char*)lk1;
  if (t0 < t1) {
    const uint32_t hf0 = tile_halves(a, t0);
    copy16(K0, ((ci32_ptr)a.col)[t0] * BLK, live16(hf0));
    load_units(dsA, hf0, (uint32_t)((cmap_ptr)a.ubase)[t0]);
    hcur = hf0;
    if (t0 + 1 < t1) {
      c1 = ((ci32_ptr)a.col)[t0 + 1];
      h1 = tile_halves(a, t0 + 1);
      u1 = (uint32_t)((cmap_ptr)a.ubase)[t0 + 1];
    }
    if (t0 + 2 < t1) {
      c2 = ((ci32_ptr)a.col)[t0 + 2];
      h2 = tile_halves(a, t0 + 2);
      u2 = (uint32_t)((cmap_ptr)a.ubase)[t0 + 2];
    }
  }
  for (int tt = t0; tt < t1; tt += 2) {
    step(tt, K0, K1, dsA, dsB);
    if (tt + 1 < t1) step(tt + 1, K1, K0, dsB, dsA);
  }
  if (j.part >= 0) {
    store_bwd_partial<D>(a, j, 32 * w + i, acc, 0, g);
    return;
  }
  store_acc_bf16<D>(make_rsrc((uint16_t*)a.out0 + j.base, a.slice_bytes), qrow, snb, acc, a.scale, g);
}

constexpr int NT8 = 512;  // dK/dV workgroup: 8 waves

// ------------------------------------------------------------------------------------------
// dK/dV with 16 keys per wave: per work item of the transposed tile list, each wave owns 16 keys
// of the block and computes, for every 32-query group of a tile in which those 16 keys have a
// valid element, S = Q K^T, P = exp2(S c2 - lse log2 e) (masked), dP - delta = dO V^T - delta,
// dS = P (dP - delta), dV^T += dO^T P and dK^T += Q^T dS (pallas_attn.py:187-215), on
// V_MFMA_F32_16X16X32_BF16. Each workgroup owns its dK/dV rows: no atomics. The waves share only
// the Q/dO tile copies and meet at the tile barriers; they hand nothing over, and each skips the
// query groups its own 16 keys have no valid element in.
//
// Register layout. S and dP are computed query-major (M = 16 queries, N = the wave's 16 keys,
// K = head_dim): lane l holds queries 4(l/16) + r (r < 4) of each 16-query half m and key
// l % 16. The contraction over queries then takes the lane's 8 values (m = 0, 1) as the 8
// consecutive K elements of its lane group, provided the other operand's K order is the same
// (queries 4g..4g+3 then 16+4g..16+4g+3): the transpose reads (ds_read_b64_tr_b16) give exactly
// that from two 4-row reads. P and dS therefore stay in registers. dV and dK accumulate
// transposed (M = 16 columns d, N = the 16 keys), so each lane ends up holding 4 consecutive
// columns of its own key per 16-column block, stored as one 8- or 16-byte write.
//
// The mask bits come from the tile list's per-lane words (fwn_tiles_prepare): for 16-key group
// kg of the block, the word of 32-row wave kg / 2, lane 32(g / 2) + 16(kg % 2) + l % 16, shifted
// right by 4(g % 2), holds element (query group c, half m, r) at bit 16c + 8m + r.
__device__ __forceinline__ f32x4 mfma16(const u32x4& a, const u32x4& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                 0, 0, 0);
}

__device__ __forceinline__ u32x4 pack8_bf16(const float (&x)[8]) {
  bf16x8 r;
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = (__bf16)x[e];
  return __builtin_bit_cast(u32x4, r);
}

// One wave's 16 keys: its K and V fragments, LDS offsets and dK^T / dV^T accumulators.
template <int D>
struct KeyWave {
  static constexpr int C = Tile<D>::C;
  static constexpr int KS = D / 32;  // K steps of the S and dP contractions
  static constexpr int NB = D / 16;  // 16-column blocks of dK^T and dV^T
  static constexpr int RS = 2 * D;   // bytes per tile row
  u32x4 kf[KS], vf[KS];              // B operands of S and dP: key krow, columns 32 s + 8 g .. +7
  uint32_t roff[KS], toff[NB];
  f32x4 dk[NB], dv[NB];

  __device__ __forceinline__ void init(const KArgs& a, const Job& j, int krow, int g, int t16) {
    const rsrc_t rK = make_rsrc((const uint16_t*)a.k + j.base, a.slice_bytes);
    const rsrc_t rV = make_rsrc((const uint16_t*)a.v + j.base, a.slice_bytes);
    const uint32_t snb = (uint32_t)a.sn * 2;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      kf[s] = bload16(rK, (uint32_t)krow * snb + (uint32_t)(64 * s + 16 * g));
      vf[s] = bload16(rV, (uint32_t)krow * snb + (uint32_t)(64 * s + 16 * g));
    }
    // LDS byte offsets within a tile, for query group 0 (group c adds 32 c rows):
    //   roff[s]: b128 row read of query row t16 (+16 m), columns 32 s + 8 g .. +7;
    //   toff[n]: transpose read, lane 4e + q of group g: row 4g + e (+16 h), columns 16 n + 4 q ..
    const int sr = swz16<C>(t16);
#pragma unroll
    for (int s = 0; s < KS; ++s) roff[s] = (uint32_t)(t16 * RS + (((4 * s + g) ^ sr) << 4));
    const int e = t16 >> 2, q = t16 & 3, trow = 4 * g + e, st = swz16<C>(trow);
#pragma unroll
    for (int n = 0; n < NB; ++n) toff[n] = (uint32_t)(trow * RS + (((2 * n + (q >> 1)) ^ st) << 4) + (q & 1) * 8);
#pragma unroll
    for (int n = 0; n < NB; ++n) {
      dk[n] = f32x4{0.f, 0.f, 0.f, 0.f};
      dv[n] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }

  // One 16-key x 32-query unit: query group c of the Q and dO tiles. `lse` and `del` point at
  // the rescaled statistics of the group's first query (-lse / scale and -delta, the initial
  // values of the S and dP accumulators, so S c2 = s c2 - lse log2 e and dP holds dP - delta).
  // Schedule (phases fenced against the compiler's scheduler): the row reads; the 16 S and dP
  // MFMAs with the 32 transpose reads of the dV and dK operands issued between them; the
  // exponentials, masks and the P pack; the 8 dV MFMAs with dS and its pack between them; the
  // 8 dK MFMAs. Each MFMA then waits for LDS once per phase, and the wave's own LDS and VALU
  // work runs while its MFMAs keep the matrix pipe busy. With `dsv`, the unit's packed dS is also
  // left there for the caller to store (the dS exchange's unit layout).
  __device__ __forceinline__ void unit(const lds_char* Q, const lds_char* O, const lds_char* lse, const lds_char* del,
                                       int c, uint64_t mw, bool full, int g, float c2, u32x4* dsv = nullptr) {
    typedef const __attribute__((address_space(3))) f32x4* cf4;
    const uint32_t cb = (uint32_t)(32 * c * RS);
    u32x4 qa[2][KS], oa[2][KS];
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        qa[m][s] = row_read(Q, roff[s] + cb + 16 * m * RS);
        oa[m][s] = row_read(O, roff[s] + cb + 16 * m * RS);
      }
    f32x4 sa[2], da[2];
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      sa[m] = *(cf4)(lse + 4 * (16 * m + 4 * g));
      da[m] = *(cf4)(del + 4 * (16 * m + 4 * g));
    }
    __builtin_amdgcn_sched_barrier(0);
    // Issue priority 1 through the MFMA phases and 0 through the exponentials: the two waves of
    // a SIMD leave each tile barrier together, and the raised priority lets the wave with MFMAs
    // to issue take the slot first (C3 dK/dV 0.773 -> 0.762 ms, c5bwd 1.485 -> 1.440 ms;
    // inverting it for waves 4-7 measured 10% slower).
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        sa[m] = mfma16(qa[m][s], kf[s], sa[m]);
        da[m] = mfma16(oa[m][s], vf[s], da[m]);
      }
    u32x2 ot[NB][2], qt[NB][2];
#pragma unroll
    for (int n = 0; n < NB; ++n)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        ot[n][h] = tr_read(O, toff[n] + cb + 16 * h * RS);
        qt[n][h] = tr_read(Q, toff[n] + cb + 16 * h * RS);
      }
#pragma unroll
    for (int i = 0; i < 4 * KS; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, NB / KS, 0);  // then transpose reads
    }
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(0);
    float p[8], ds[8];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      p[r] = fast_exp2(sa[0][r] * c2);
      p[4 + r] = fast_exp2(sa[1][r] * c2);
    }
    {
      // Applied to every unit, fully valid ones included (their bits are all set): a branch here
      // would split the phase and let the compiler sink the transpose reads past it.
      const uint32_t w32 = (uint32_t)(mw >> (32 * (c >> 1)));
#pragma unroll
      for (int i = 0; i < 8; ++i)
        p[i] = keep_or_zero(p[i], __builtin_amdgcn_sbfe(w32, (uint32_t)(16 * (c & 1) + 8 * (i >> 2) + (i & 3)), 1u));
    }
    const u32x4 pb = pack8_bf16(p);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int n = 0; n < NB; ++n) dv[n] = mfma16(u32x4{ot[n][0][0], ot[n][0][1], ot[n][1][0], ot[n][1][1]}, pb, dv[n]);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      ds[r] = p[r] * da[0][r];
      ds[4 + r] = p[4 + r] * da[1][r];
    }
    const u32x4 db = pack8_bf16(ds);
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);  // one dV MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, 2, 1);  // then dS / pack VALU work
    }
    __builtin_amdgcn_sched_barrier(0);
    if (dsv) *dsv = db;
#pragma unroll
    for (int n = 0; n < NB; ++n) dk[n] = mfma16(u32x4{qt[n][0][0], qt[n][0][1], qt[n][1][0], qt[n][1][1]}, db, dk[n]);
    __builtin_amdgcn_s_setprio(0);
  }

  // Query groups of the tile in which these 16 keys have a valid element (a wave-uniform set,
  // from this lane's mask word `mw`), and those in which all 512 elements are valid.
  static __device__ __forceinline__ void live_units(uint64_t mw, uint32_t& live, uint32_t& full) {
    live = 0u;
    full = 0u;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint32_t b8 = (uint32_t)(mw >> (16 * c)) & 0x0F0Fu;
      if (__builtin_amdgcn_ballot_w64(b8 != 0u) != 0u) live |= 1u << c;
      if (__builtin_amdgcn_ballot_w64(b8 != 0x0F0Fu) == 0u) full |= 1u << c;
    }
  }

  // dK^T / dV^T block n: lane l holds columns 16 n + 4 g .. +3 of key krow (row `prow` of the
  // block in a partial slot).
  __device__ __forceinline__ void store(const KArgs& a, const Job& j, int krow, int prow, int g) const {
    if (j.part >= 0) {
      const rsrc_t r = part_slot<D>(a, j);
#pragma unroll
      for (int n = 0; n < NB; ++n) {
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, dk[n]), r,
                                               (int)((uint32_t)(prow * D + 16 * n + 4 * g) * 4), 0, 0);
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, dv[n]), r,
                                               (int)((uint32_t)((128 + prow) * D + 16 * n + 4 * g) * 4), 0, 0);
      }
      return;
    }
    const rsrc_t rdk = make_rsrc((uint16_t*)a.out0 + j.base, a.slice_bytes);
    const rsrc_t rdv = make_rsrc((uint16_t*)a.out1 + j.base, a.slice_bytes);
    const uint32_t snb = (uint32_t)a.sn * 2;
#pragma unroll
    for (int n = 0; n < NB; ++n) {
      u32x2 wk, wv;
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) {
        const __bf16 k0 = (__bf16)(dk[n][2 * h2] * a.scale), k1 = (__bf16)(dk[n][2 * h2 + 1] * a.scale);
        const __bf16 v0 = (__bf16)dv[n][2 * h2], v1 = (__bf16)dv[n][2 * h2 + 1];
        wk[h2] = (uint32_t)__builtin_bit_cast(uint16_t, k0) | ((uint32_t)__builtin_bit_cast(uint16_t, k1) << 16);
        wv[h2] = (uint32_t)__builtin_bit_cast(uint16_t, v0) | ((uint32_t)__builtin_bit_cast(uint16_t, v1) << 16);
      }
      const uint32_t off = (uint32_t)krow * snb + (uint32_t)(2 * (16 * n + 4 * g));
      __builtin_amdgcn_raw_buffer_store_b64(wk, rdk, (int)off, 0, 0);
      __builtin_amdgcn_raw_buffer_store_b64(wv, rdv, (int)off, 0, 0);
    }
  }
};

// 8 waves, one workgroup per CU, the Q/dO tiles double-buffered: one barrier per tile.
//
// With DS (the bf16 backward with the dS exchange), every unit's dS also goes to HBM as one 1 KB
// unit, 16 bytes per lane in the order the registers hold it (DsUnit). Units are numbered over
// the forward tile list: tile tf's live halves (bit 8c + kg for query group c and 16-key group kg)
// hold units ubase[tf] + (rank of the bit among the set bits); tmap gives (ubase, halves) of the
// forward tile for each tile of this transposed list. The host checks that this list is the exact
// transpose of the forward one, so the units this wave computes are exactly that tile's set bits.
// A unit's store is issued at the start of the wave's next unit (or after its final tile), so the
// vmcnt(0) before each tile barrier never waits for a store issued just before it; the stores are
// non-temporal (nothing in this kernel reads them; allocating them in L2 would evict Q/dO tiles).
template <int D, bool DS = false>
__global__ void __launch_bounds__(NT8, 1) dkv16_kernel(KArgs a) {
  constexpr int TB = Tile<D>::BYTES;
  __shared__ __attribute__((aligned(1024))) char lds0[2 * TB + 1536];  // Q | dO | lse[128] | gap | delta[128]
  __shared__ __attribute__((aligned(1024))) char lds1[2 * TB + 1536];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);  // keys 16 wid .. 16 wid + 15 of the block
  const int g = lane >> 4, t16 = lane & 15;
  const Job j = decode_job(a);
  if (j.skip) return;  // an empty entry of the order table
  const uint32_t snb = (uint32_t)a.sn * 2, osnb = (uint32_t)a.osn * 2;
  const rsrc_t rQ = make_rsrc((const uint16_t*)a.q + j.base, a.slice_bytes);
  const rsrc_t rO = make_rsrc((const uint16_t*)a.dout + j.obase, a.oslice_bytes);
  const rsrc_t rL = make_rsrc(a.lse + stat_index(a, j, 0), (uint32_t)a.n * 4);
  const rsrc_t rD = make_rsrc(a.delta + stat_index(a, j, 0), (uint32_t)a.n * 4);
  const int krow = j.blk * BLK + 16 * wid + t16;
  KeyWave<D> kw;
  kw.init(a, j, krow, g, t16);

  // Tile copies, in one of three modes per wave: 0, waves 0-3 copy Q and waves 4-7 dO; 1, this
  // wave issues both shares of its SIMD pair (waves wid % 4 and wid % 4 + 4: the Q and dO ops of
  // class wid % 4); 2, none (its partner is in mode 1). The tile's 128 lse and delta (two
  // branch-free full-wave copies; out-of-range halves read zeros into the gap) go with wave 0 in
  // mode 0 and with pair 0's copier otherwise; the same wave rescales them at the start of the
  // tile's step, after waiting for its own copies (pair 0's copier has the fewer units, so its
  // rescale delays the barrier least: C5-shape dK/dV -1%).
  TileDma<D, true> dma, dmaQ, dmaO;
  dma.init(wid & 3, lane, wid < 4 ? snb : osnb);
  dmaQ.init(wid & 3, lane, snb);
  dmaO.init(wid & 3, lane, osnb);
  constexpr uint32_t kPastEnd = 0x7FFFFFF0u;
  auto stats_wave = [&](int mode) { return mode == 0 ? wid == 0 : (mode == 1 && (wid & 3) == 0); };
  bool stats_cur = false;  // this wave copied the current tile's lse and delta (it rescales them)
  auto issue = [&](int qb, lds_char* buf, uint32_t copy, int mode) {
    if (mode == 0) {
      if (wid < 4) {
        dma.issue(rQ, buf, wid, qb * BLK, snb, copy);
      } else {
        dma.issue(rO, buf + TB, wid - 4, qb * BLK, osnb, copy);
      }
    } else if (mode == 1) {
      dmaQ.issue(rQ, buf, wid & 3, qb * BLK, snb, copy);
      dmaO.issue(rO, buf + TB, wid & 3, qb * BLK, osnb, copy);
    }
    if (stats_wave(mode)) {
      const uint32_t vo = (uint32_t)(qb * BLK + 4 * (lane & 31)) * 4;
      lds_char* stats = buf + 2 * TB;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rL, (__attribute__((address_space(3))) void*)stats, 16,
                                               (int)(lane < 32 ? vo : kPastEnd), 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rD, (__attribute__((address_space(3))) void*)(stats + 512), 16,
                                               (int)(lane < 32 ? kPastEnd : vo), 0, 0, 0);
    }
  };
  const uint64_t* mword = key_mask_words(a, wid, g, t16);
  const int mshift = 4 * (g & 1);

  // dS exchange state: the unit computed last (its dS in dsv, its byte offset in pend; pend =
  // ds_slice_bytes means no unit yet, and that store falls outside the buffer range) and the
  // forward tile's (ubase, halves) for the current tile, read at the end of the previous tile's
  // step (a scalar load pending when the units start would make their first LDS wait wait for it
  // too).
  rsrc_t rS;
  u32x4 dsv = {0u, 0u, 0u, 0u};
  uint32_t pend = 0u, ubc = 0u, hfc = 0u;
  typedef const __attribute__((address_space(4))) uint32_t* cmap_ptr;
  if constexpr (DS) {
    rS = make_rsrc(a.ds + (int64_t)j.bh * (a.ds_slice_bytes >> 1), a.ds_slice_bytes);
    pend = a.ds_slice_bytes;
  }
  // The unit's offset goes into the per-lane offset (voffset), which the buffer unit checks
  // against the slice size (soffset is not checked): with pend = ds_slice_bytes every lane's
  // 16 bytes lie past the range and the store writes nothing. A branch on pend instead measured
  // 2% slower.
  auto store_ds = [&]() {
    if constexpr (DS) __builtin_amdgcn_raw_buffer_store_b128(dsv, rS, (int)(16u * lane + pend), 0, kNonTemporal);
  };

  // The next tile's group bits and column block are read a tile ahead (scalar loads), so issuing
  // its copy right after the barrier waits for neither.
  auto tile_step = [&](int tt, int t1, lds_char* cur, lds_char* nxt, uint64_t& mnext, uint32_t& gnext,
                       int& cnext) {
    const int t = __builtin_amdgcn_readfirstlane(tt);
    bool stats_nxt = false;
    wait_vmem();  // this wave's part of tile t and its mask word
    const uint64_t mw = mnext >> mshift;
    if (stats_cur) {
      // lse -> -lse / scale and delta -> -delta, the initial values of the S and dP accumulators.
      __attribute__((address_space(3))) f32x4* x =
          (__attribute__((address_space(3))) f32x4*)(cur + 2 * TB + (lane < 32 ? 0 : 512) + 16 * lane);
      float m = lane < 32 ? a.nlse_mul : -1.f;
      asm volatile("" : "+v"(m));
      *x = *x * m;
    }
    __syncthreads();  // tile t is in LDS; every wave is done with tile t - 1 (buffer nxt)
    if (t + 1 < t1) {
      mnext = mword[(int64_t)(t + 1) * 256];
      // With the dS map, every wave's unit count in this tile is known from the forward tile's
      // half bits (bit 8c + kg: query group c, 16-key group kg). The wave of each SIMD pair with
      // fewer units issues the pair's whole copy and the other goes straight to its units: the
      // SIMD's copy ops queue behind each other whichever wave issues them (the older wave's
      // first), so the queueing then lands on the wave with less to compute (C3 dK/dV 0.636 ->
      // 0.606 ms, C5 shape -2 to -3%).
      int mode = 0;
      if constexpr (DS) {
        const int s = wid & 3;
        const uint32_t ns = (uint32_t)__builtin_popcount(hfc >> s & 0x01010101u);
        const uint32_t ns4 = (uint32_t)__builtin_popcount(hfc >> (s + 4) & 0x01010101u);
        mode = ((wid < 4) == (ns <= ns4)) ? 1 : 2;
      }
      issue(cnext, nxt, any_rows(gnext), mode);
      stats_nxt = stats_wave(mode);
    }
    if (t + 2 < t1) {
      gnext = tile_groups(a, t + 2);
      cnext = ((ci32_ptr)a.col)[t + 2];
    }
    uint32_t live, full;
    KeyWave<D>::live_units(mw, live, full);
    const lds_char* stats = cur + 2 * TB;
#pragma unroll
    for (int c = 0; c < 4; ++c)
      if (live >> c & 1u) {
        if constexpr (DS) {
          store_ds();
          kw.unit(cur, cur + TB, stats + 128 * c, stats + 1024 + 128 * c, c, mw, full >> c & 1u, g, a.c2, &dsv);
          const uint32_t bit = 8u * c + (uint32_t)wid;
          pend = (ubc + (uint32_t)__builtin_popcount(hfc & ((1u << bit) - 1u))) * 1024u;
        } else {
          kw.unit(cur, cur + TB, stats + 128 * c, stats + 1024 + 128 * c, c, mw, full >> c & 1u, g, a.c2);
        }
      }
    if constexpr (DS) {
      if (t + 1 < t1) {
        ubc = ((cmap_ptr)a.tmap)[2 * (t + 1)];
        hfc = ((cmap_ptr)a.tmap)[2 * (t + 1) + 1];
      }
    }
    stats_cur = stats_nxt;
  };

  int t0, t1;
  tile_range(a, j, t0, t1);
  uint64_t mnext = 0;
  uint32_t gnext = 0u;
  int cnext = 0;
  lds_char* b0 = (lds_char*)lds0;
  lds_char* b1 = (lds_char*)lds1;
  if (t0 < t1) {
    mnext = mword[(int64_t)t0 * 256];
    if (t0 + 1 < t1) {
      gnext = tile_groups(a, t0 + 1);
      cnext = ((ci32_ptr)a.col)[t0 + 1];
    }
    if constexpr (DS) {
      ubc = ((cmap_ptr)a.tmap)[2 * t0];
      hfc = ((cmap_ptr)a.tmap)[2 * t0 + 1];
    }
    issue(((ci32_ptr)a.col)[t0], b0, any_rows(tile_groups(a, t0)), 0);
    stats_cur = wid == 0;
  }
  for (int tt = t0; tt < t1; tt += 2) {
    tile_step(tt, t1, b0, b1, mnext, gnext, cnext);
    if (tt + 1 < t1) tile_step(tt + 1, t1, b1, b0, mnext, gnext, cnext);
  }
  store_ds();  // the last unit's dS (none when the wave computed no unit)
  kw.store(a, j, krow, 16 * wid + t16, g);
}

template <int D>
hipError_t launch_d(Kind kind, const KArgs& a, hipStream_t stream) {
  const dim3 grid((unsigned)job_count(a)), block(NT);
  switch (kind) {
    case Kind::kFwd: hipLaunchKernelGGL(fwd_kernel<D>, grid, block, 0, stream, a); break;
    case Kind::kDq: hipLaunchKernelGGL(dq_kernel<D>, grid, block, 0, stream, a); break;
    case Kind::kDkv: hipLaunchKernelGGL((dkv16_kernel<D, false>), grid, dim3(NT8), 0, stream, a); break;
    case Kind::kDkvDs: hipLaunchKernelGGL((dkv16_kernel<D, true>), grid, dim3(NT8), 0, stream, a); break;
    case Kind::kDqDs: hipLaunchKernelGGL(dq_ds_kernel<D>, grid, block, 0, stream, a); break;
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
