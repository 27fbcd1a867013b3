// Combine passes of split blocks: a block whose tile run was cut into several work items has one
// float32 partial slot per item; these kernels merge a block's slots into the outputs.
//
// Forward: each slot holds unnormalised O rows with the row max m_c (log2 domain) and row sum
// l_c of its key range; O = sum_c 2^(m_c - M) O_c / sum_c 2^(m_c - M) l_c with M = max_c m_c,
// and lse = (M + log2 L) ln 2, the same online-softmax merge the forward kernel applies between
// tiles (pallas_attn.py:128-141). dQ, dK, dV: partial sums over disjoint tile ranges, added and
// scaled as the kernels scale their direct outputs (pallas_attn.py:184, 214-215).
//
// Each thread handles 8 consecutive columns of one row; a (split block, batch, head) takes
// 128 * D / 8 threads, D / 16 workgroups of 256.
#include "attn_device.h"

namespace fwn {
namespace {

using namespace dev;

constexpr int kThreads = 256;

struct Split {
  int blk, p0, np, b, h, bh;
  bool ok;
};

__device__ __forceinline__ Split decode_split(const KArgs& a, int job) {
  Split s;
  const int bh_count = a.batch * a.heads;
  const int idx = job / bh_count;
  s.bh = job - idx * bh_count;
  const ci32_ptr e = (ci32_ptr)a.split + 3 * idx;
  s.blk = e[0];
  s.p0 = e[1];
  s.np = e[2];
  s.b = s.bh / a.heads;
  s.h = s.bh - s.b * a.heads;
  s.ok = (unsigned)s.blk < (unsigned)a.n_blocks && s.p0 >= 0 && s.np > 0 && s.p0 + s.np <= a.n_parts;
  return s;
}

template <int D>
__device__ __forceinline__ const float* slot_ptr(const KArgs& a, const Split& s, int c) {
  return a.work + ((int64_t)(s.p0 + c) * a.batch * a.heads + s.bh) * (int64_t)(128 * (2 * D + 2));
}

// Stores 4 float32 values as the output dtype at element offset `off` of `base`.
template <typename T>
__device__ __forceinline__ void store4(void* base, int64_t off, const f32x4& x) {
  if constexpr (sizeof(T) == 4) {
    *(f32x4*)((float*)base + off) = x;
  } else {
    u32x2 w;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const __bf16 lo = (__bf16)x[2 * h], hi = (__bf16)x[2 * h + 1];
      w[h] = (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
    }
    *(u32x2*)((uint16_t*)base + off) = w;
  }
}

// Workgroups per (split block, batch, head) and this thread's (row, first column).
template <int D>
struct Cell {
  static constexpr int CH = D / 8;                 // 8-column chunks per row
  static constexpr int WGS = 128 * CH / kThreads;  // D / 16
  int job, r, d;
  __device__ __forceinline__ Cell() {
    job = blockIdx.x / WGS;
    const int id = (blockIdx.x - job * WGS) * kThreads + threadIdx.x;
    r = id / CH;
    d = (id - r * CH) * 8;
  }
};

template <typename T, int D>
__global__ void __launch_bounds__(kThreads) fwd_combine_kernel(KArgs a) {
  const Cell<D> cell;
  const Split s = decode_split(a, cell.job);
  const int r = cell.r, d = cell.d;
  const int row = s.blk * BLK + r;
  if (!s.ok || row >= a.n) return;
  float M = -__builtin_inff();
  for (int c = 0; c < s.np; ++c) M = fmaxf(M, slot_ptr<D>(a, s, c)[128 * D + r]);
  const float base = M == -__builtin_inff() ? 0.f : M;
  float L = 0.f;
  f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = acc0;
  for (int c = 0; c < s.np; ++c) {
    const float* p = slot_ptr<D>(a, s, c);
    const float wgt = fast_exp2(p[128 * D + r] - base);
    L += p[128 * D + 128 + r] * wgt;
    acc0 += wgt * *(const f32x4*)(p + r * D + d);
    acc1 += wgt * *(const f32x4*)(p + r * D + d + 4);
  }
  const float inv = L > 0.f ? 1.f / L : 0.f;
  const int64_t out_off = (int64_t)s.b * a.osb + (int64_t)s.h * a.osh + (int64_t)row * a.osn + d;
  store4<T>(a.out0, out_off, acc0 * inv);
  store4<T>(a.out0, out_off + 4, acc1 * inv);
  if (d == 0 && a.lse_out)
    a.lse_out[((int64_t)s.b * a.heads + s.h) * a.n + row] = (M + __builtin_amdgcn_logf(fmaxf(L, 1e-30f))) * LN2;
}

// dQ (one output, scaled) or dK/dV (two outputs: dK scaled, dV not).
template <typename T, int D, int OUTS>
__global__ void __launch_bounds__(kThreads) bwd_combine_kernel(KArgs a) {
  const Cell<D> cell;
  const Split s = decode_split(a, cell.job);
  const int r = cell.r, d = cell.d;
  const int row = s.blk * BLK + r;
  if (!s.ok || row >= a.n) return;
  const int64_t out_off = (int64_t)s.b * a.sb + (int64_t)s.h * a.sh + (int64_t)row * a.sn + d;
#pragma unroll
  for (int o = 0; o < OUTS; ++o) {
    f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = acc0;
    for (int c = 0; c < s.np; ++c) {
      const float* p = slot_ptr<D>(a, s, c) + (o * 128 + r) * D + d;
      acc0 += *(const f32x4*)p;
      acc1 += *(const f32x4*)(p + 4);
    }
    const float mul = o == 0 ? a.scale : 1.f;
    void* out = o == 0 ? a.out0 : a.out1;
    store4<T>(out, out_off, acc0 * mul);
    store4<T>(out, out_off + 4, acc1 * mul);
  }
}

template <typename T, int D>
hipError_t launch_td(Kind kind, const KArgs& a, hipStream_t stream) {
  const dim3 grid((unsigned)a.n_split * (unsigned)(a.batch * a.heads) * (unsigned)Cell<D>::WGS), block(kThreads);
  switch (kind) {
    case Kind::kFwdCombine: hipLaunchKernelGGL((fwd_combine_kernel<T, D>), grid, block, 0, stream, a); break;
    case Kind::kDqCombine: hipLaunchKernelGGL((bwd_combine_kernel<T, D, 1>), grid, block, 0, stream, a); break;
    case Kind::kDkvCombine: hipLaunchKernelGGL((bwd_combine_kernel<T, D, 2>), grid, block, 0, stream, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <typename T>
hipError_t launch_t(Kind kind, int head_dim, const KArgs& a, hipStream_t stream) {
  switch (head_dim) {
    case 32: return launch_td<T, 32>(kind, a, stream);
    case 64: return launch_td<T, 64>(kind, a, stream);
    case 128: return launch_td<T, 128>(kind, a, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_combine(Kind kind, int dtype, int head_dim, const KArgs& a, hipStream_t stream) {
  if (a.n_split <= 0) return hipSuccess;
  return dtype == 0 ? launch_t<float>(kind, head_dim, a, stream) : launch_t<uint16_t>(kind, head_dim, a, stream);
}

}  // namespace fwn
