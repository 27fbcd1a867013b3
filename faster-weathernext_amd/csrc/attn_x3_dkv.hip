// dK/dV of the bf16x3 backward (FWN_PREC_BF16X3) with the dS exchange. The split K and V rows
// (128 registers) and the dK^T / dV^T accumulators (128) fill the 256 VGPRs of its one wave per
// SIMD; the compiler keeps the streamed operands and the S / dP accumulators partly in AGPRs.
//
// Reference: pallas_attn.py:187-215 (the dK/dV kernel), 336-341 (precision selection).
#include "attn_x3.h"

namespace fwn {
namespace {

using namespace dev;

// dK/dV, float32 tensors, bf16x3 products, the dS exchange (pallas_attn.py:187-215). Four waves,
// one workgroup per CU; wave w owns keys 32 w .. + 31 of the key block and keeps their K and V
// rows split in registers (the B operands of S = Q K^T and dP = dO V^T) and dK^T, dV^T in
// accumulators. The transposed list's (tile, query group) steps stream through two group buffers
// as in the forward: Q and dO as split planes plus the group's 32 lse (times log2 e) and delta.
// Per live 32 x 32 group: S and dP (3 D/16 MFMAs each, dP's accumulator starting at -delta),
// P = exp2(S c2 - lse log2 e) masked, dS = P (dP - delta), dV^T += dO^T P and dK^T += Q^T dS
// (3 D/16 each, the transposed operands by ds_read_b64_tr_b16).
//
// With DS every group's dS goes to HBM as one 4 KB unit: chunk 64 k + L (16 bytes) holds, for dQ
// lane L (query L % 32, g = L / 32), keys 16 c + 8 g .. + 7 of plane p (k = 2 p + c; p = 0 hi,
// 1 lo). This lane holds one key and 16 queries, so the wave transposes through its own LDS stage
// ([plane][query][key] bf16, 80-byte rows: conflict-free 16-byte row reads) before four 16-byte
// non-temporal stores per lane. Units are numbered as in the float32 exchange (rank of group bit
// 4 c + w of the forward tile, from tmap).
template <int D, bool DS>
__global__ void __launch_bounds__(NT, 1) dkv_x3_kernel(KArgs a) {
  constexpr int GB = X3Dma<D>::GB;
  constexpr int SB = 4 * GB;  // Q hi | Q lo | dO hi | dO lo | lse [32], 0 [32] | delta [32], 0 [32]
  constexpr int SROW = 80, SPLANE = 32 * SROW;
  __shared__ __attribute__((aligned(1024))) char gb0[SB + 512];
  __shared__ __attribute__((aligned(1024))) char gb1[SB + 512];
  __shared__ __attribute__((aligned(16))) char stage[DS ? 4 * 2 * SPLANE : 16];
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i = lane & 31, g = lane >> 5;
  const Job j = decode_job(a);
  const int64_t xbase = (int64_t)j.bh * a.n * (2 * D);
  const rsrc_t rQ = make_rsrc(a.xa + xbase, a.xslice_bytes);
  const rsrc_t rO = make_rsrc(a.xb + xbase, a.xslice_bytes);
  const rsrc_t rL = make_rsrc(a.lse + stat_index(a, j, 0), (uint32_t)a.n * 4);
  const rsrc_t rD = make_rsrc(a.delta + stat_index(a, j, 0), (uint32_t)a.n * 4);
  const uint32_t snb = (uint32_t)a.sn * 4;
  const int krow = j.blk * BLK + 32 * w + i;
  u32x4 kh[D / 16], kl[D / 16], vh[D / 16], vl[D / 16];
  load_frag_x3<D>(kh, kl, make_rsrc((const float*)a.k + j.base, a.slice_bytes), krow, snb, g);
  load_frag_x3<D>(vh, vl, make_rsrc((const float*)a.v + j.base, a.slice_bytes), krow, snb, g);
  Off<D> off;
  off.init(lane);
  X3Dma<D> dma;
  dma.init(w, lane);
  f32x16 dk[D / 32], dv[D / 32];
#pragma unroll
  for (int db = 0; db < D / 32; ++db) {
    dk[db] = zero16();
    dv[db] = zero16();
  }
  rsrc_t rS;
  if constexpr (DS) rS = make_rsrc(a.ds + (int64_t)j.bh * (a.ds_slice_bytes >> 1), a.ds_slice_bytes);
  typedef const __attribute__((address_space(4))) uint32_t* cmap_ptr;

  // Query group c of the tile from group buffer buf; `ub`, `gw`: the forward tile's first unit and
  // group word (DS).
  auto group = [&](int c, const lds_char* buf, u32x2 mb, uint32_t ub, uint32_t gw) {
    const lds_char* lq = buf;
    const lds_char* lo = buf + 2 * GB;
    typedef const __attribute__((address_space(3))) float* cfp;
    const cfp lse = (cfp)(buf + SB);
    const cfp del = (cfp)(buf + SB + 256);
    // S and dP, the four row reads (Q hi, Q lo, dO hi, dO lo) of k-step k + 1 issued before the
    // six MFMAs of step k: at most two steps of operands are live.
    auto rows = [&](u32x4 (&x)[4], int k) {
      x[0] = row_read(lq, off.row[k]);
      x[1] = row_read(lq + GB, off.row[k]);
      x[2] = row_read(lo, off.row[k]);
      x[3] = row_read(lo + GB, off.row[k]);
    };
    u32x4 ra[2][4];
    rows(ra[0], 0);
    f32x16 s = zero16(), dp;
#pragma unroll
    for (int r = 0; r < 16; ++r) dp[r] = -del[element_col(0, r, g)];
#pragma unroll
    for (int k = 0; k < D / 16; ++k) {
      if (k + 1 < D / 16) rows(ra[(k + 1) & 1], k + 1);
      __builtin_amdgcn_sched_barrier(0);
      s = mfma_x3(ra[k & 1][0], ra[k & 1][1], kh[k], kl[k], s);
      dp = mfma_x3(ra[k & 1][2], ra[k & 1][3], vh[k], vl[k], dp);
      __builtin_amdgcn_sched_barrier(0);
    }
    // dV^T += dO^T P and dK^T += Q^T dS by (column block db, query half c2) pairs; the four
    // transpose reads of a pair are issued one pair ahead, the first during the exponentials.
    auto trs = [&](u32x4 (&x)[4], int pr) {
      const int db = pr >> 1, c2 = pr & 1;
      x[0] = tr_operand<D>(lo, off, db, 0, c2);
      x[1] = tr_operand<D>(lo + GB, off, db, 0, c2);
      x[2] = tr_operand<D>(lq, off, db, 0, c2);
      x[3] = tr_operand<D>(lq + GB, off, db, 0, c2);
    };
    u32x4 ta[2][4];
    trs(ta[0], 0);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float p = fast_exp2(fmaf(s[r], a.c2, -lse[element_col(0, r, g)]));
      p = keep_or_zero(p, elem_keep(mb, c, r));
      s[r] = p;
      dp[r] = p * dp[r];
    }
    u32x4 ph[2], pl[2], dh[2], dl[2];
#pragma unroll
    for (int c2 = 0; c2 < 2; ++c2) {
      split_acc(s, c2, ph[c2], pl[c2]);
      split_acc(dp, c2, dh[c2], dl[c2]);
    }
    constexpr int NP = 2 * (D / 32);
#pragma unroll
    for (int pr = 0; pr < NP; ++pr) {
      if (pr + 1 < NP) trs(ta[(pr + 1) & 1], pr + 1);
      __builtin_amdgcn_sched_barrier(0);
      const int db = pr >> 1, c2 = pr & 1;
      const u32x4(&x)[4] = ta[pr & 1];
      dv[db] = mfma_x3(x[0], x[1], ph[c2], pl[c2], dv[db]);
      dk[db] = mfma_x3(x[2], x[3], dh[c2], dl[c2], dk[db]);
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (DS) {
      const uint32_t bit = 4u * (uint32_t)c + (uint32_t)w;
      if (gw >> bit & 1u) {
        const uint32_t u = ub + (uint32_t)__builtin_popcount(gw & 0xffffu & ((1u << bit) - 1u));
        __attribute__((address_space(3))) char* st = (__attribute__((address_space(3))) char*)stage + w * 2 * SPLANE;
        // The stage is written as 16-bit and read as 128-bit values: compiler barriers keep this
        // unit's writes after the previous unit's reads and before this unit's reads (the LDS
        // executes one wave's accesses in order).
        asm volatile("" ::: "memory");
        // This lane's key i, queries 16 c2 + 8 g + e, into column i of the stage.
#pragma unroll
        for (int pl2 = 0; pl2 < 2; ++pl2)
#pragma unroll
          for (int c2 = 0; c2 < 2; ++c2) {
            const u32x4 x = pl2 ? dl[c2] : dh[c2];
#pragma unroll
            for (int e = 0; e < 8; ++e)
              *(__attribute__((address_space(3))) uint16_t*)(st + pl2 * SPLANE + (16 * c2 + 8 * g + e) * SROW + 2 * i) =
                  (uint16_t)(x[e >> 1] >> (16 * (e & 1)));
          }
        asm volatile("" ::: "memory");
        // Lane (query i, g): keys 16 cc + 8 g .. + 7 of its row, per plane.
#pragma unroll
        for (int pl2 = 0; pl2 < 2; ++pl2)
#pragma unroll
          for (int cc = 0; cc < 2; ++cc) {
            const u32x4 x = *(const __attribute__((address_space(3))) u32x4*)(st + pl2 * SPLANE + i * SROW +
                                                                               2 * (16 * cc + 8 * g));
            __builtin_amdgcn_raw_buffer_store_b128(x, rS, 16 * (64 * (2 * pl2 + cc) + lane), (int)(u * 4096u),
                                                   kNonTemporal);
          }
      }
    }
  };

  int t0, t1;
  tile_range(a, j, t0, t1);
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
  // Step (t, c): the group's Q and dO planes and, by wave 0, its lse and delta (lanes 32-63 read
  // zeros into the gaps).
  auto copy = [&](lds_char* buf, int t, int c) {
    const int row0 = ((ci32_ptr)a.col)[t] * BLK + 32 * c;
    dma.issue(rQ, rO, buf, row0, w);
    if (w == 0) {
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
  u32x2 mbc = {0u, 0u}, mbn = {0u, 0u};
  if (vc) {
    copy(b0, tc, cc);
    mbc = tile_bits(a, tc, w, lane);
    vn = take(tn, cn);
  }
  auto step = [&](lds_char* cur, lds_char* nxt) {
    wait_vmem();  // this wave's part of the current step (wave 0: the statistics too) and its mask bits
    if (w == 0 && lane < 8) {
      // lse -> lse * log2(e), the form the exponent takes
      __attribute__((address_space(3))) f32x4* x = (__attribute__((address_space(3))) f32x4*)(cur + SB + 16 * lane);
      *x = *x * LOG2E;
    }
    __syncthreads();  // the step landed; every wave is done with the previous step's buffer
    if (vn) {
      copy(nxt, tn, cn);
      mbn = tn != tc ? tile_bits(a, tn, w, lane) : mbc;
    }
    const uint32_t gt = tile_groups(a, tc);
    uint32_t ub = 0u, gw = 0u;
    if constexpr (DS) {
      ub = ((cmap_ptr)a.tmap)[2 * tc];
      gw = ((cmap_ptr)a.tmap)[2 * tc + 1];
    }
    if (gt >> (4 * w + cc) & 1u) group(cc, cur, mbc, ub, gw);
    tc = tn;
    cc = cn;
    mbc = mbn;
    vc = vn;
    vn = vc && take(tn, cn);
  };
  while (vc) {
    step(b0, b1);
    if (!vc) break;
    step(b1, b0);
  }
  if (j.part >= 0) {
    store_bwd_partial<D>(a, j, 32 * w + i, dk, 0, g);
    store_bwd_partial<D>(a, j, 32 * w + i, dv, 1, g);
    return;
  }
  store_acc_f32<D>(make_rsrc((float*)a.out0 + j.base, a.slice_bytes), krow, snb, dk, a.scale, g);
  store_acc_f32<D>(make_rsrc((float*)a.out1 + j.base, a.slice_bytes), krow, snb, dv, 1.f, g);
}

template <int D>
hipError_t launch_d(const KArgs& a, hipStream_t stream) {
  const dim3 grid((unsigned)a.n_items * (unsigned)(a.batch * a.heads)), block(NT);
  hipLaunchKernelGGL((dkv_x3_kernel<D, true>), grid, block, 0, stream, a);
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
