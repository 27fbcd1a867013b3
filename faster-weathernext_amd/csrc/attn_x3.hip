// The bf16x3 (split-precision) kernels for float32 tensors (FWN_PREC_BF16X3): the split pass,
// the forward and dQ from dS (dK/dV is in attn_x3_dkv.hip). Every product is formed from bf16
// parts on V_MFMA_F32_32X32X16_BF16: x = hi + lo with hi = bf16(x) and lo = bf16(x - hi), and
// a*b = ah*bh + ah*bl + al*bh in fp32 accumulation (al*bl, about 2^-18 of the product, is
// dropped). Each operand then carries about 16-17 significant bits instead of bf16's 8 (TF32 has
// 11), at three bf16 MFMAs per product: 5.3x the fp32-MFMA rate. This is the role of the
// reference's TF32 and TF32_TF32_F32_X3 dots (pallas_attn.py:336-343) on a target without TF32
// matrix instructions.
//
// The operands that stream through LDS (forward: K, V; dK/dV: Q, dO; dQ: K) are split once per
// call by split_x3_kernel into [batch * heads][n][2][D] bf16 (hi row, then lo row) and copied by
// 32-row group; the operands a wave keeps in registers (forward: Q; dK/dV: its K and V rows) are
// split when loaded; P and dS are split in registers.
//
// The backward is the dS exchange (5 contractions per tile): dK/dV computes S, dP, dV, dK and
// writes each 32 x 32 dS group as hi and lo bf16 (4 KB, the float32 exchange's unit size and
// numbering), in the dQ kernel's operand order; dQ = scale * dS K reads it.
//
// Reference: pallas_attn.py:112-141 (forward kernel), 161-215 (backward kernels), 317-354
// (precision selection).
#include "attn_x3.h"

namespace fwn {
namespace {

using namespace dev;

struct SplitArgs {
  const float* src;
  uint16_t* dst;
  int64_t sb, sn, sh;  // element strides of src
  int32_t batch, n, heads, d;
};

// One thread per 8 consecutive elements of a row: 32 bytes read, 16 bytes of hi and 16 of lo
// written. dst is [batch * heads][n][2][d]: (batch, head) slices of n split rows.
__global__ void __launch_bounds__(256) split_x3_kernel(SplitArgs s) {
  const uint32_t per_row = (uint32_t)s.d / 8u;
  const uint32_t idx = blockIdx.x * 256u + threadIdx.x;
  const uint32_t rows = (uint32_t)s.batch * (uint32_t)s.heads * (uint32_t)s.n;
  if (idx >= rows * per_row) return;
  const uint32_t r = idx / per_row, c = idx - r * per_row;
  const uint32_t bh = r / (uint32_t)s.n, node = r - bh * (uint32_t)s.n;
  const uint32_t b = bh / (uint32_t)s.heads, h = bh - b * (uint32_t)s.heads;
  const float* p = s.src + (int64_t)b * s.sb + (int64_t)node * s.sn + (int64_t)h * s.sh + 8 * c;
  const f32x4 x0 = *(const f32x4*)p, x1 = *(const f32x4*)(p + 4);
  const float x[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
  u32x4 hi, lo;
  split8(x, hi, lo);
  uint16_t* q = s.dst + (int64_t)r * 2 * s.d + 8 * c;
  *(u32x4*)q = hi;
  *(u32x4*)(q + s.d) = lo;
}

// Forward, float32 tensors, bf16x3 products: two workgroups per CU, streamed by 32-key group
// (the steps are the work item's (tile, key group) pairs in which some wave has a valid element).
// Each step's four planes (32 KB at D = 128) go into one of two group buffers; the copy of step
// s + 1 runs while step s is computed, one barrier per step. Per live group a wave issues 3 D/16
// MFMAs for S^T = K Q^T and 3 D/16 for O^T += V^T P^T, with the online softmax of the bf16
// forward between them (lazy rescale, masks skipped for fully valid groups).
template <int D>
__global__ void __launch_bounds__(NT, 2) fwd_x3_kernel(KArgs a) {
  constexpr int GB = X3Dma<D>::GB;
  __shared__ __attribute__((aligned(1024))) char gb0[4 * GB];
  __shared__ __attribute__((aligned(1024))) char gb1[4 * GB];
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i = lane & 31, g = lane >> 5;
  const Job j = decode_job(a);
  if (j.skip) return;  // an empty entry of the order table
  const int64_t xbase = (int64_t)j.bh * a.n * (2 * D);
  const rsrc_t rK = make_rsrc(a.xa + xbase, a.xslice_bytes);
  const rsrc_t rV = make_rsrc(a.xb + xbase, a.xslice_bytes);
  const int qrow = j.blk * BLK + 32 * w + i;
  u32x4 qh[D / 16], ql[D / 16];
  load_frag_x3<D>(qh, ql, make_rsrc((const float*)a.q + j.base, a.slice_bytes), qrow, (uint32_t)a.sn * 4, g);
  Off<D> off;
  off.init(lane);
  X3Dma<D> dma;
  dma.init(w, lane);
  f32x16 o[D / 32];
#pragma unroll
  for (int db = 0; db < D / 32; ++db) o[db] = zero16();
  SoftmaxState st{-__builtin_inff(), 0.f};

  // Key group sb of a tile from group buffer buf (mask bits mb; `full`: every element valid).
  auto group = [&](int sb, const lds_char* buf, u32x2 mb, bool full) {
    u32x4 kh[D / 16], kl[D / 16];
#pragma unroll
    for (int s = 0; s < D / 16; ++s) {
      kh[s] = row_read(buf, off.row[s]);
      kl[s] = row_read(buf + GB, off.row[s]);
    }
    __builtin_amdgcn_sched_barrier(0);
    f32x16 s[1];
    s[0] = zero16();
#pragma unroll
    for (int k = 0; k < D / 16; ++k) s[0] = mfma_x3(kh[k], kl[k], qh[k], ql[k], s[0]);
    // V's transpose reads are in flight during the mask and the softmax.
    u32x4 vh[D / 32][2], vl[D / 32][2];
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        vh[db][c] = tr_operand<D>(buf + 2 * GB, off, db, 0, c);
        vl[db][c] = tr_operand<D>(buf + 3 * GB, off, db, 0, c);
      }
    if (!full) {
#pragma unroll
      for (int r = 0; r < 16; ++r) s[0][r] = keep_or_ninf(s[0][r], elem_keep(mb, sb, r));
    }
    float corr;
    if (softmax_live<1>(s, 1u, st, a.c2, corr)) {
#pragma unroll
      for (int db = 0; db < D / 32; ++db) o[db] *= corr;
    }
    u32x4 ph[2], pl[2];
    split_acc(s[0], 0, ph[0], pl[0]);
    split_acc(s[0], 1, ph[1], pl[1]);
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
      for (int c = 0; c < 2; ++c) o[db] = mfma_x3(vh[db][c], vl[db][c], ph[c], pl[c], o[db]);
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
  auto copy = [&](lds_char* buf, int t, int c) { dma.issue(rK, rV, buf, ((ci32_ptr)a.col)[t] * BLK + 32 * c, w); };
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
  // One step: step (tc, cc) is in `cur`; the copy of step (tn, cn) goes into `nxt`.
  auto step = [&](lds_char* cur, lds_char* nxt) {
    wait_vmem();      // this wave's part of the current step (and its mask bits)
    __syncthreads();  // the step landed; every wave is done with the previous step's buffer
    if (vn) {
      copy(nxt, tn, cn);
      mbn = tn != tc ? tile_bits(a, tn, w, lane) : mbc;
    }
    const uint32_t gt = tile_groups(a, tc);
    if (gt >> (4 * w + cc) & 1u) group(cc, cur, mbc, gt >> (16 + 4 * w + cc) & 1u);
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
  const float ltot = st.l + __shfl_xor(st.l, 32);
  if (j.part >= 0) {
    store_fwd_partial<D>(a, j, 32 * w + i, o, st.m, ltot, g);
    return;
  }
  const float inv = ltot > 0.f ? 1.f / ltot : 0.f;
  store_acc_f32<D>(make_rsrc((float*)a.out0 + j.obase, a.oslice_bytes), qrow, (uint32_t)a.osn * 4, o, inv, g);
  if (g == 0) write_lse(a, j, qrow, st, ltot);
}

// dQ, float32 tensors, bf16x3 products, from the dS units of dkv16_x3_kernel: per work item
// of the forward list, dQ^T += K^T dS^T over each wave's live 32 x 32 groups (pallas_attn.py:
// 177-184 with dS from the dK/dV pass). Per tile half (key groups 2h, 2h + 1) the split K rows go
// into one of two half buffers (planes K hi, K lo of each group: 32 KB at D = 128), two workgroups
// per CU; a half's units (four 16-byte non-temporal loads per lane: the B operands' hi and lo
// parts) are loaded with its rows, so the barrier that publishes the rows covers them.
template <int D>
__global__ void __launch_bounds__(NT, 2) dq_x3_ds_kernel(KArgs a) {
  constexpr int GB = X3Dma<D>::GB;
  __shared__ __attribute__((aligned(1024))) char hb0[4 * GB];
  __shared__ __attribute__((aligned(1024))) char hb1[4 * GB];
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i = lane & 31, g = lane >> 5;
  const Job j = decode_job(a);
  if (j.skip) return;  // an empty entry of the order table
  const int64_t xbase = (int64_t)j.bh * a.n * (2 * D);
  const rsrc_t rK = make_rsrc(a.xa + xbase, a.xslice_bytes);
  // The same slice from row 32 on: planes 2, 3 of a half hold its second key group.
  const uint32_t skip = 32u * 4u * D;
  const rsrc_t rK2 = make_rsrc(a.xa + xbase + 32 * 2 * D, a.xslice_bytes > skip ? a.xslice_bytes - skip : 0u);
  const rsrc_t rS = make_rsrc(a.ds + (int64_t)j.bh * (a.ds_slice_bytes >> 1), a.ds_slice_bytes);
  const int qrow = j.blk * BLK + 32 * w + i;
  Off<D> off;
  off.init(lane);
  X3Dma<D> dma;
  dma.init(w, lane);
  f32x16 acc[D / 32];
#pragma unroll
  for (int db = 0; db < D / 32; ++db) acc[db] = zero16();
  typedef const __attribute__((address_space(4))) uint32_t* cmap_ptr;

  // This wave's units of tile half h (key groups 2h + x: group bits 4 w + 2 h + x).
  auto load_units = [&](u32x4 (&dst)[2][4], uint32_t gw, uint32_t ub, int h) {
    const uint32_t b0 = 4u * (uint32_t)w + 2u * (uint32_t)h;
    uint32_t u = ub + (uint32_t)__builtin_popcount(gw & 0xffffu & ((1u << b0) - 1u));
#pragma unroll
    for (int x = 0; x < 2; ++x)
      if (gw >> (b0 + x) & 1u) {
#pragma unroll
        for (int k = 0; k < 4; ++k)
          // The unit's offset in the per-lane offset: checked against the slice size.
          dst[x][k] = __builtin_amdgcn_raw_buffer_load_b128(rS, (int)(16u * (64 * k + lane) + u * 4096u), 0, kNonTemporal);
        ++u;
      }
  };
  // Key group x of the half buffer hb (planes 2x, 2x + 1), with its unit d.
  auto group = [&](int x, const lds_char* hb, const u32x4 (&d)[4]) {
    u32x4 th[D / 32][2], tl[D / 32][2];
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        th[db][c] = tr_operand<D>(hb + 2 * x * GB, off, db, 0, c);
        tl[db][c] = tr_operand<D>(hb + (2 * x + 1) * GB, off, db, 0, c);
      }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
      for (int c = 0; c < 2; ++c) acc[db] = mfma_x3(th[db][c], tl[db][c], d[c], d[2 + c], acc[db]);
  };
  auto copy = [&](lds_char* hb, int kb, int h, uint32_t live) {
    const uint32_t planes = (live >> (2 * h) & 1u ? 3u : 0u) | (live >> (2 * h + 1) & 1u ? 12u : 0u);
    dma.issue(rK, rK2, hb, kb * BLK + 64 * h, w, planes);
  };

  int t0, t1;
  tile_range(a, j, t0, t1);
  u32x4 dsA[2][4], dsB[2][4];  // units of the current tile's half 0 and half 1
  uint32_t gcur = 0u, ucur = 0u;
  lds_char* h0 = (lds_char*)hb0;
  lds_char* h1 = (lds_char*)hb1;
  if (t0 < t1) {
    gcur = tile_groups(a, t0);
    ucur = ((cmap_ptr)a.ubase)[t0];
    copy(h0, ((ci32_ptr)a.col)[t0], 0, any_rows(gcur));
    load_units(dsA, gcur, ucur, 0);
  }
  for (int tt = t0; tt < t1; ++tt) {
    const int t = __builtin_amdgcn_readfirstlane(tt);
    const int kb = ((ci32_ptr)a.col)[t];
    const uint32_t gt = gcur, ut = ucur;
    const uint32_t live = gt >> (4 * w) & 15u;
    wait_vmem();      // this wave's part of half 0 of tile t and its units
    __syncthreads();  // half 0 landed; every wave is done with half 1 of tile t - 1
    copy(h1, kb, 1, any_rows(gt));
    load_units(dsB, gt, ut, 1);
    if (t + 1 < t1) {
      gcur = tile_groups(a, t + 1);
      ucur = ((cmap_ptr)a.ubase)[t + 1];
    }
    __builtin_amdgcn_sched_barrier(0);
    if (live & 1u) group(0, h0, dsA[0]);
    __builtin_amdgcn_sched_barrier(0);
    if (live & 2u) group(1, h0, dsA[1]);
    __builtin_amdgcn_sched_barrier(0);
    wait_vmem();      // this wave's part of half 1 and its units
    __syncthreads();  // half 1 landed; every wave is done with half 0
    if (t + 1 < t1) {
      copy(h0, ((ci32_ptr)a.col)[t + 1], 0, any_rows(gcur));
      load_units(dsA, gcur, ucur, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (live & 4u) group(0, h1, dsB[0]);
    __builtin_amdgcn_sched_barrier(0);
    if (live & 8u) group(1, h1, dsB[1]);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (j.part >= 0) {
    store_bwd_partial<D>(a, j, 32 * w + i, acc, 0, g);
    return;
  }
  store_acc_f32<D>(make_rsrc((float*)a.out0 + j.base, a.slice_bytes), qrow, (uint32_t)a.sn * 4, acc, a.scale, g);
}

template <int D>
hipError_t launch_d(Kind kind, const KArgs& a, hipStream_t stream) {
  const dim3 grid((unsigned)job_count(a)), block(NT);
  switch (kind) {
    case Kind::kFwd: hipLaunchKernelGGL(fwd_x3_kernel<D>, grid, block, 0, stream, a); break;
    case Kind::kDqDs: hipLaunchKernelGGL(dq_x3_ds_kernel<D>, grid, block, 0, stream, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_x3(Kind kind, int head_dim, const KArgs& a, hipStream_t stream) {
  if (kind == Kind::kDkvDs) return launch_x3_dkv(head_dim, a, stream);
  switch (head_dim) {
    case 32: return launch_d<32>(kind, a, stream);
    case 64: return launch_d<64>(kind, a, stream);
    case 128: return launch_d<128>(kind, a, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_split_x3(const float* src, int64_t sb, int64_t sn, int64_t sh, int batch, int n, int heads,
                           int head_dim, uint16_t* dst, hipStream_t stream) {
  SplitArgs s{src, dst, sb, sn, sh, batch, n, heads, head_dim};
  const uint64_t threads = (uint64_t)batch * heads * n * (head_dim / 8);
  hipLaunchKernelGGL(split_x3_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream, s);
  return hipGetLastError();
}

}  // namespace fwn
