// Split-precision forward for float32 tensors (FWN_PREC_BF16X3): every product of S = Q K^T and
// O = P V is formed from bfloat16 parts on V_MFMA_F32_32X32X16_BF16, x = hi + lo with
// hi = bf16(x) and lo = bf16(x - hi), as hi*hi + hi*lo + lo*hi in fp32 accumulation (the lo*lo
// term is below fp32 rounding of the sum). Each operand then carries about 16 significant bits
// instead of bf16's 8 (TF32 has 11), at three bf16 MFMAs per product: 5.3x the fp32-MFMA rate.
// This is the role of the reference's TF32_TF32_F32_X3 dots under "highest" precision
// (pallas_attn.py:336-341): an fp32-accurate forward on the matrix cores' fast type.
//
// K and V are split once per call by split_x3_kernel into [batch * heads][n][2][D] bf16 (hi row,
// then lo row), which the forward streams into LDS by 32-key group; Q is split in registers at
// the start of each work item; P is split in registers after the softmax.
//
// Reference: pallas_attn.py:112-141 (forward kernel), 317-354 (precision selection).
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

// Copy of one step's 32 split K rows and 32 split V rows into a group buffer of four 32-row planes
// (K hi, K lo, V hi, V lo; each [32][D] bf16, chunks swizzled as the bf16 tiles). Each wave-wide
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

  __device__ __forceinline__ void issue(rsrc_t rK, rsrc_t rV, lds_char* buf, int row0, int w) const {
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
      const uint32_t src = (uint32_t)(row0 + RPO * sub) * XROW + voff + (uint32_t)(plane & 1) * (2 * D);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          m < D / 32 ? rK : rV,
          (__attribute__((address_space(3))) void*)(uintptr_t)(base + (uint32_t)(plane * GB + sub * 1024)), 16,
          (int)src, 0, 0, 0);
    }
  }
};

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
  const int64_t xbase = (int64_t)j.bh * a.n * (2 * D);
  const rsrc_t rK = make_rsrc(a.kx + xbase, a.xslice_bytes);
  const rsrc_t rV = make_rsrc(a.vx + xbase, a.xslice_bytes);
  const int qrow = j.blk * BLK + 32 * w + i;
  u32x4 qh[D / 16], ql[D / 16];
  {
    const rsrc_t rQ = make_rsrc((const float*)a.q + j.base, a.slice_bytes);
    const uint32_t qoff = (uint32_t)qrow * ((uint32_t)a.sn * 4) + (uint32_t)(32 * g);
#pragma unroll
    for (int s = 0; s < D / 16; ++s) {
      const f32x4 x0 = __builtin_bit_cast(f32x4, bload16(rQ, qoff + 64 * s));
      const f32x4 x1 = __builtin_bit_cast(f32x4, bload16(rQ, qoff + 64 * s + 16));
      const float x[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
      split8(x, qh[s], ql[s]);
    }
  }
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

template <int D>
hipError_t launch_d(Kind kind, const KArgs& a, hipStream_t stream) {
  const dim3 grid((unsigned)a.n_items * (unsigned)(a.batch * a.heads)), block(NT);
  switch (kind) {
    case Kind::kFwd: hipLaunchKernelGGL(fwd_x3_kernel<D>, grid, block, 0, stream, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_x3(Kind kind, int head_dim, const KArgs& a, hipStream_t stream) {
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
