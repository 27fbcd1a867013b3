// dK/dV of the bf16x3 backward (FWN_PREC_BF16X3) with the dS exchange: 16 keys per wave on
// V_MFMA_F32_16X16X32_BF16, so that a wave's split K and V rows (64 registers) and its dK^T / dV^T
// accumulators (64) leave room for a second wave per SIMD.
//
// Reference: pallas_attn.py:187-215 (the dK/dV kernel), 336-341 (precision selection).
#include "attn_x3.h"

namespace fwn {
namespace {

using namespace dev;

constexpr int NT4 = 256;  // 4 waves

// 16x16x32 bf16 MFMA and its three-part product (cross terms first, then hi * hi).
__device__ __forceinline__ f32x4 mfma16(const u32x4& a, const u32x4& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                 0, 0, 0);
}

__device__ __forceinline__ f32x4 mfma16_x3(const u32x4& ah, const u32x4& al, const u32x4& bh, const u32x4& bl,
                                           f32x4 c) {
  c = mfma16(al, bh, c);
  c = mfma16(ah, bl, c);
  return mfma16(ah, bh, c);
}

// X3Dma for NW waves and the 16-key kernel's tile swizzle (swz16): instruction k = w + NW m of the
// 4 NI of a step fills rows RPO (k % NI) .. of plane k / NI. The swizzle depends on row % 8, the
// same for every instruction of one wave (RPO NW is a multiple of 8).
template <int D, int NW>
struct X3DmaW {
  static constexpr int C = D / 8;
  static constexpr int RPO = 1024 / (2 * D);
  static constexpr int NI = 32 / RPO;
  static constexpr int GB = 32 * 2 * D;
  static constexpr int XROW = 4 * D;
  uint32_t voff;

  __device__ __forceinline__ void init(int w, int lane) {
    const int row = RPO * (w % NI) + lane / C;
    voff = (uint32_t)(lane / C) * XROW + (uint32_t)(((lane % C) ^ swz16<C>(row)) << 4);
  }

  __device__ __forceinline__ void issue(rsrc_t rA, rsrc_t rB, lds_char* buf, int row0, int w) const {
    uint32_t base = (uint32_t)(uintptr_t)buf;
    asm volatile("" : "+s"(base));
#pragma unroll
    for (int m = 0; m < 4 * NI / NW; ++m) {
      const int k = w + NW * m, plane = k / NI, sub = k % NI;
      const uint32_t src = (uint32_t)(row0 + RPO * sub) * XROW + voff + (uint32_t)(plane & 1) * (2 * D);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          plane < 2 ? rA : rB,
          (__attribute__((address_space(3))) void*)(uintptr_t)(base + (uint32_t)(plane * GB + sub * 1024)), 16,
          (int)src, 0, 0, 0);
    }
  }
};

// dK/dV, float32 tensors, bf16x3 products, the dS exchange, 16 keys per wave, two waves per SIMD.
// Each work item's 128 keys are split between two 4-wave workgroups of 64 keys (75 KB of LDS
// each), two per CU on the same XCD, each streaming only the query groups its own keys need and
// meeting at barriers of its own. The wave of 16-key group kg owns keys 16 kg .. + 15 of the key
// block and keeps their K and V rows split in registers (64) and dK^T, dV^T (64); lane l holds
// key l % 16 and queries 4 g + r, 16 + 4 g + r (g = l / 16, r < 4) of a 32-query group, as the
// bf16 16-key kernel. Steps are the transposed list's (tile, query group) pairs, streamed through
// two group buffers (Q hi, Q lo, dO hi, dO lo planes, swizzled by swz16, plus the group's
// statistics).
// A unit (16 keys x 32 queries) streams its operand reads one MFMA step ahead: the four row reads
// of (k-step, query half) before the previous pair's six MFMAs, the four transpose reads of a
// 16-column block before the previous block's six.
//
// dS: a 32 x 32 unit of the float32 exchange belongs to the two waves of its 32-key group; the wave
// of group kg writes 16-key chunk kg % 2 of both planes (chunk 64 (2 p + kg % 2) + L for dQ lane
// L), through a per-wave LDS stage ([plane][query][16 keys] bf16, 32-byte rows: conflict-free
// 16-byte reads). A wave whose 16 keys have no valid element in a unit the map has writes zeros
// for its chunk.
template <int D>
__global__ void __launch_bounds__(NT4, 2) dkv16_x3_kernel(KArgs a) {
  using Dma = X3DmaW<D, 4>;
  constexpr int GB = Dma::GB;
  constexpr int SB = 4 * GB;  // Q hi | Q lo | dO hi | dO lo | -lse/scale [32], 0 [32] | -delta [32], 0 [32]
  constexpr int KS = D / 32;  // k-steps of S and dP
  constexpr int NB = D / 16;  // 16-column blocks of dK^T and dV^T
  constexpr int RS = 2 * D;   // bytes per plane row
  constexpr int C = D / 8;
  __shared__ __attribute__((aligned(1024))) char gb0[SB + 512];
  __shared__ __attribute__((aligned(1024))) char gb1[SB + 512];
  __shared__ __attribute__((aligned(16))) char stage[4 * 2048];
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
  const int64_t xbase = (int64_t)j.bh * a.n * (2 * D);
  const rsrc_t rQ = make_rsrc(a.xa + xbase, a.xslice_bytes);
  const rsrc_t rO = make_rsrc(a.xb + xbase, a.xslice_bytes);
  const rsrc_t rL = make_rsrc(a.lse + stat_index(a, j, 0), (uint32_t)a.n * 4);
  const rsrc_t rD = make_rsrc(a.delta + stat_index(a, j, 0), (uint32_t)a.n * 4);
  const rsrc_t rS = make_rsrc(a.ds + (int64_t)j.bh * (a.ds_slice_bytes >> 1), a.ds_slice_bytes);
  const uint32_t snb = (uint32_t)a.sn * 4;
  const int krow = j.blk * BLK + 16 * kg + t16;
  // K and V rows of this lane's key, columns 32 s + 8 g .. + 7, split.
  u32x4 kh[KS], kl[KS], vh[KS], vl[KS];
  {
    const rsrc_t rK = make_rsrc((const float*)a.k + j.base, a.slice_bytes);
    const rsrc_t rV = make_rsrc((const float*)a.v + j.base, a.slice_bytes);
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const uint32_t off = (uint32_t)krow * snb + (uint32_t)(128 * s + 32 * g);
      const f32x4 k0 = __builtin_bit_cast(f32x4, bload16(rK, off)), k1 = __builtin_bit_cast(f32x4, bload16(rK, off + 16));
      const f32x4 v0 = __builtin_bit_cast(f32x4, bload16(rV, off)), v1 = __builtin_bit_cast(f32x4, bload16(rV, off + 16));
      const float xk[8] = {k0[0], k0[1], k0[2], k0[3], k1[0], k1[1], k1[2], k1[3]};
      const float xv[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
      split8(xk, kh[s], kl[s]);
      split8(xv, vh[s], vl[s]);
    }
  }
  // LDS offsets within a plane, formed where they are used (a register each would not fit):
  // roff(s) the row read of query row t16 (+16 m), columns 32 s + 8 g ..; toff(n) the transpose
  // read of lane 4 e + q of group g: row 4 g + e (+16 h), columns 16 n + 4 q ...
  const int sr = swz16<C>(t16);
  const uint32_t rbase = (uint32_t)(t16 * RS);
  const int te = t16 >> 2, tq = t16 & 3, trow = 4 * g + te, tsw = swz16<C>(trow);
  const uint32_t tbase = (uint32_t)(trow * RS + (tq & 1) * 8);
  auto roff = [&](int s) { return rbase + (uint32_t)(((4 * s + g) ^ sr) << 4); };
  auto toff = [&](int n) { return tbase + (uint32_t)(((2 * n + (tq >> 1)) ^ tsw) << 4); };
  Dma dma;
  dma.init(wid, lane);
  f32x4 dk[NB], dv[NB];
#pragma unroll
  for (int n = 0; n < NB; ++n) {
    dk[n] = f32x4{0.f, 0.f, 0.f, 0.f};
    dv[n] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  typedef const __attribute__((address_space(4))) uint32_t* cmap_ptr;
  typedef const __attribute__((address_space(3))) f32x4* cf4;
  const uint64_t* mword = key_mask_words(a, kg, g, t16);
  const int mshift = 4 * (g & 1);
  __attribute__((address_space(3))) char* stw = (__attribute__((address_space(3))) char*)stage + wid * 2048;

  // The dS chunk of a unit: `have` false writes zeros (no valid element for these 16 keys).
  auto store_chunk = [&](bool have, const u32x4& dh, const u32x4& dl, uint32_t u) {
    const int i = lane & 31, gq = lane >> 5;
    u32x4 y[2] = {u32x4{0u, 0u, 0u, 0u}, u32x4{0u, 0u, 0u, 0u}};
    if (have) {
      asm volatile("" ::: "memory");
#pragma unroll
      for (int pl = 0; pl < 2; ++pl) {
        const u32x4 x = pl ? dl : dh;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int qr = 16 * (e >> 2) + 4 * g + (e & 3);
          *(__attribute__((address_space(3))) uint16_t*)(stw + pl * 1024 + qr * 32 + 2 * t16) =
              (uint16_t)(x[e >> 1] >> (16 * (e & 1)));
        }
      }
      asm volatile("" ::: "memory");
#pragma unroll
      for (int pl = 0; pl < 2; ++pl) y[pl] = *(const __attribute__((address_space(3))) u32x4*)(stw + pl * 1024 + i * 32 + 16 * gq);
      asm volatile("" ::: "memory");
    }
#pragma unroll
    for (int pl = 0; pl < 2; ++pl)  // the unit's offset in the per-lane offset: checked against the slice size
      __builtin_amdgcn_raw_buffer_store_b128(y[pl], rS, (int)(16u * (64 * (2 * pl + (wid & 1)) + lane) + u * 4096u), 0,
                                             kNonTemporal);
  };

  // Unit: query group c of the group buffer buf (mask word mw of this lane); split dS into dh, dl.
  auto unit = [&](int c, const lds_char* buf, uint64_t mw, u32x4& dh, u32x4& dl) {
    const lds_char* qh = buf;
    const lds_char* oh = buf + 2 * GB;
    f32x4 sa[2], da[2];
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      sa[m] = *(cf4)(buf + SB + 4 * (16 * m + 4 * g));
      da[m] = *(cf4)(buf + SB + 256 + 4 * (16 * m + 4 * g));
    }
    auto rows = [&](u32x4 (&x)[4], int it) {
      const int s = it >> 1, m = it & 1;
      const uint32_t o = roff(s) + 16 * m * RS;
      x[0] = row_read(qh, o);
      x[1] = row_read(qh + GB, o);
      x[2] = row_read(oh, o);
      x[3] = row_read(oh + GB, o);
    };
    u32x4 rd[2][4];
    rows(rd[0], 0);
    __builtin_amdgcn_s_setprio(1);  // MFMA phases at issue priority 1, the exponentials at 0
#pragma unroll
    for (int it = 0; it < 2 * KS; ++it) {
      if (it + 1 < 2 * KS) rows(rd[(it + 1) & 1], it + 1);
      __builtin_amdgcn_sched_barrier(0);
      const int s = it >> 1, m = it & 1;
      const u32x4(&x)[4] = rd[it & 1];
      sa[m] = mfma16_x3(x[0], x[1], kh[s], kl[s], sa[m]);
      da[m] = mfma16_x3(x[2], x[3], vh[s], vl[s], da[m]);
      __builtin_amdgcn_sched_barrier(0);
    }
    auto trs = [&](u32x4 (&x)[4], int n) {
      const uint32_t o = toff(n);
      const u32x2 a0 = tr_read(oh, o), a1 = tr_read(oh, o + 16 * RS);
      const u32x2 b0 = tr_read(oh + GB, o), b1 = tr_read(oh + GB, o + 16 * RS);
      const u32x2 c0 = tr_read(qh, o), c1 = tr_read(qh, o + 16 * RS);
      const u32x2 d0 = tr_read(qh + GB, o), d1 = tr_read(qh + GB, o + 16 * RS);
      x[0] = u32x4{a0[0], a0[1], a1[0], a1[1]};
      x[1] = u32x4{b0[0], b0[1], b1[0], b1[1]};
      x[2] = u32x4{c0[0], c0[1], c1[0], c1[1]};
      x[3] = u32x4{d0[0], d0[1], d1[0], d1[1]};
    };
    u32x4 tb[2][4];
    trs(tb[0], 0);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(0);
    float p[8], ds[8];
    const uint32_t w32 = (uint32_t)(mw >> (32 * (c >> 1)));
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float se = e < 4 ? sa[0][e & 3] : sa[1][e & 3];
      const float de = e < 4 ? da[0][e & 3] : da[1][e & 3];
      const float pe = keep_or_zero(fast_exp2(se * a.c2),
                                    __builtin_amdgcn_sbfe(w32, (uint32_t)(16 * (c & 1) + 8 * (e >> 2) + (e & 3)), 1u));
      p[e] = pe;
      ds[e] = pe * de;
    }
    u32x4 ph, pl;
    split8(p, ph, pl);
    split8(ds, dh, dl);
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int n = 0; n < NB; ++n) {
      if (n + 1 < NB) trs(tb[(n + 1) & 1], n + 1);
      __builtin_amdgcn_sched_barrier(0);
      const u32x4(&x)[4] = tb[n & 1];
      dv[n] = mfma16_x3(x[0], x[1], ph, pl, dv[n]);
      dk[n] = mfma16_x3(x[2], x[3], dh, dl, dk[n]);
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
  auto copy = [&](lds_char* buf, int t, int c) {
    const int row0 = ((ci32_ptr)a.col)[t] * BLK + 32 * c;
    dma.issue(rQ, rO, buf, row0, wid);
    if (wid == 0) {
      const int so = lane < 32 ? (row0 + lane) * 4 : (int)kPastEnd;
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
      // lse -> -lse / scale and delta -> -delta: the initial values of the S and dP accumulators
      // (S c2 = s c2 - lse log2 e).
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
    // The wave's 16 keys have a valid element in query group cc: some lane's bits of the group
    // (16 c + 8 m + r, shifted by 4 (g % 2)) are set.
    const uint64_t mw = mwc >> mshift;
    const bool live = __builtin_amdgcn_ballot_w64((((uint32_t)(mw >> (16 * cc))) & 0x0F0Fu) != 0u) != 0u;
    const uint32_t ub = ((cmap_ptr)a.tmap)[2 * tc];
    const uint32_t gw = ((cmap_ptr)a.tmap)[2 * tc + 1];
    const uint32_t bit = 4u * (uint32_t)cc + (uint32_t)(kg >> 1);
    const bool have_unit = (gw >> bit & 1u) != 0u;
    const uint32_t u = ub + (uint32_t)__builtin_popcount(gw & 0xffffu & ((1u << bit) - 1u));
    // One store path after the unit (a store inside the unit's branch and another beside it made
    // the register allocator place dK^T / dV^T differently on each path and copy them every step).
    u32x4 dh = {0u, 0u, 0u, 0u}, dl = {0u, 0u, 0u, 0u};
    if (live) unit(cc, cur, mw, dh, dl);
    if (have_unit) store_chunk(live, dh, dl, u);
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

template <int D>
hipError_t launch_d(const KArgs& a, hipStream_t stream) {
  // Two workgroups per item, laid out in blocks of 16 ids (8 items x 2 halves).
  const dim3 grid(16u * (((unsigned)job_count(a) + 7u) / 8u));
  hipLaunchKernelGGL((dkv16_x3_kernel<D>), grid, dim3(NT4), 0, stream, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_x3_dkv(int head_dim, const KArgs& a, hipStream_t stream) {
  switch (head_dim) {
    case 32: return launch_d<32>(a, stream);
    case 64: return launch_d<64>(a, stream);
    case 128: return launch_d<128>(a, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace fwn
