// Row permutation passes fused with layer norms (gfx950): the gather of the node features into
// Hilbert order before the mesh transformer's layers together with the first block's layer
// norm, and the final layer norm with its per-member affine together with the scatter back
// (patch.py:244, 274-276, 288-292). The second pass without a permutation is each block's
// conditioned layer norm, optionally with the residual add in front of it (patch.py:240-253).
//
// Both passes are HBM-bound streaming: one wave per row, 16 bytes per lane per load, so each
// wave-wide load or store covers 1 KB of one row. A row stays in registers between its
// statistics and its outputs, so every byte is read once. Statistics are float32: the mean
// first, then the biased variance of the centred values, both as fixed-order wave sums.
#include "rows_kernels.h"

#include "fwn_attn.h"

namespace fwn {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;  // rows per workgroup, one per wave

// Bit reinterpretation of a vector element. The element is passed by value: clang's
// __builtin_bit_cast applied to a subscripted ext_vector lvalue (v[e]) reads element 0 for
// every e (seen with this ROCm's hipcc), so it is never applied to v[e] directly.
__device__ __forceinline__ float as_float(uint32_t u) { return __builtin_bit_cast(float, u); }

template <typename T>
struct Vec;

template <>
struct Vec<float> {
  static constexpr int E = 4;  // elements per 16-byte vector
  __device__ __forceinline__ static void unpack(const u32x4& v, float (&f)[E]) {
#pragma unroll
    for (int e = 0; e < 4; ++e) f[e] = as_float(v[e]);
  }
  __device__ __forceinline__ static u32x4 pack(const float (&f)[E]) {
    return u32x4{__builtin_bit_cast(uint32_t, f[0]), __builtin_bit_cast(uint32_t, f[1]),
                 __builtin_bit_cast(uint32_t, f[2]), __builtin_bit_cast(uint32_t, f[3])};
  }
};

template <>
struct Vec<uint16_t> {  // bfloat16 bits
  static constexpr int E = 8;
  __device__ __forceinline__ static void unpack(const u32x4& v, float (&f)[E]) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      f[2 * k] = as_float(v[k] << 16);
      f[2 * k + 1] = as_float(v[k] & 0xffff0000u);
    }
  }
  __device__ __forceinline__ static u32x4 pack(const float (&f)[E]) {  // round to nearest even
    u32x4 v;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t lo = __builtin_bit_cast(uint16_t, (__bf16)f[2 * k]);
      const uint32_t hi = __builtin_bit_cast(uint16_t, (__bf16)f[2 * k + 1]);
      v[k] = lo | (hi << 16);
    }
    return v;
  }
};

// Output rows are written once and not read again by the pass: non-temporal stores stream them
// past the caches (gather pass at [1, 40962, 768] float32: 74.5 -> 56.3 us, 6.7 TB/s).
__device__ __forceinline__ void store16(void* p, const u32x4& v) { __builtin_nontemporal_store(v, (u32x4*)p); }

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
  return x;
}

// Loads one row (VPL vectors per lane, vector lane + 64k) and returns its mean and 1/std. With
// `row2`, the row is row + row2, added in float32 and rounded once to T (as a separate
// elementwise add would store it); v then holds that sum and the statistics are the sum's.
template <typename T, int VPL>
__device__ __forceinline__ void load_row(const T* row, bool ok, int nv, int channels, float eps, int lane,
                                         u32x4 (&v)[VPL], float (&f)[VPL][Vec<T>::E], float& mean, float& rstd,
                                         const T* row2 = nullptr) {
  constexpr int E = Vec<T>::E;
  float sum = 0.f;
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int idx = lane + 64 * k;
    v[k] = u32x4{0u, 0u, 0u, 0u};
    if (ok && idx < nv) v[k] = *(const u32x4*)(row + (size_t)idx * E);
    Vec<T>::unpack(v[k], f[k]);
    if (row2) {
      u32x4 w = u32x4{0u, 0u, 0u, 0u};
      if (ok && idx < nv) w = *(const u32x4*)(row2 + (size_t)idx * E);
      float g[E];
      Vec<T>::unpack(w, g);
#pragma unroll
      for (int e = 0; e < E; ++e) f[k][e] += g[e];
      v[k] = Vec<T>::pack(f[k]);
      Vec<T>::unpack(v[k], f[k]);
    }
#pragma unroll
    for (int e = 0; e < E; ++e) sum += f[k][e];
  }
  mean = wave_sum(sum) / (float)channels;
  float sq = 0.f;
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    if (lane + 64 * k >= nv) continue;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const float c = f[k][e] - mean;
      sq = fmaf(c, c, sq);
    }
  }
  const float var = wave_sum(sq) / (float)channels;
  rstd = __builtin_amdgcn_rsqf(var + eps);
}

template <typename T, int VPL>
__global__ void __launch_bounds__(64 * kWaves) gather_norm_kernel(RowArgs a) {
  constexpr int E = Vec<T>::E;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (row >= (int64_t)a.batch * a.n) return;  // whole waves leave together
  const int64_t b = row / a.n, i = row - b * a.n;
  const int64_t src = a.perm[i];
  const bool ok = src >= 0 && src < a.n;
  const size_t c = (size_t)a.channels;
  const int nv = a.channels / E;
  u32x4 v[VPL];
  float f[VPL][E];
  float mean, rstd;
  load_row<T, VPL>((const T*)a.x + (size_t)(b * a.n + (ok ? src : 0)) * c, ok, nv, a.channels, a.eps, lane, v, f,
                   mean, rstd);
  T* xo = (T*)a.x_out + (size_t)row * c;
  T* no = a.norm_out ? (T*)a.norm_out + (size_t)row * c : nullptr;
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int idx = lane + 64 * k;
    if (idx >= nv) continue;
    store16(xo + (size_t)idx * E, v[k]);
    if (no) {
      float y[E];
#pragma unroll
      for (int e = 0; e < E; ++e) y[e] = (f[k][e] - mean) * rstd;
      store16(no + (size_t)idx * E, Vec<T>::pack(y));
    }
  }
}

// ADD: a.addend is added to x first and the sum written to a.x_out (a compile-time switch, so
// the plain pass carries no test for it).
template <typename T, int VPL, bool ADD>
__global__ void __launch_bounds__(64 * kWaves) norm_scatter_kernel(RowArgs a) {
  constexpr int E = Vec<T>::E;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (row >= (int64_t)a.batch * a.n) return;
  const int64_t b = row / a.n, i = row - b * a.n;
  const int64_t dst = a.perm ? a.perm[i] : i;  // no permutation: the conditioned layer norm alone
  if (dst < 0 || dst >= a.n) return;
  const size_t c = (size_t)a.channels;
  const int nv = a.channels / E;
  u32x4 v[VPL];
  float f[VPL][E];
  float mean, rstd;
  load_row<T, VPL>((const T*)a.x + (size_t)row * c, true, nv, a.channels, a.eps, lane, v, f, mean, rstd,
                   ADD ? (const T*)a.addend + (size_t)row * c : nullptr);
  if constexpr (ADD) {  // the sum x + addend, in place of x's row (the whole row is in registers)
    T* so = (T*)a.x_out + (size_t)row * c;
#pragma unroll
    for (int k = 0; k < VPL; ++k)
      if (lane + 64 * k < nv) store16(so + (size_t)(lane + 64 * k) * E, v[k]);
  }
  T* o = (T*)a.out + (size_t)(b * a.n + dst) * c;
  const float* mul = a.mul ? a.mul + (size_t)b * c : nullptr;
  const float* add = a.add ? a.add + (size_t)b * c : nullptr;
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int idx = lane + 64 * k;
    if (idx >= nv) continue;
    float y[E];
#pragma unroll
    for (int e = 0; e < E; ++e) y[e] = (f[k][e] - mean) * rstd;
    if (mul) {
#pragma unroll
      for (int q = 0; q < E / 4; ++q) {
        const u32x4 m = *(const u32x4*)(mul + (size_t)idx * E + 4 * q);
#pragma unroll
        for (int e = 0; e < 4; ++e) y[4 * q + e] *= as_float(m[e]);
      }
    }
    if (add) {
#pragma unroll
      for (int q = 0; q < E / 4; ++q) {
        const u32x4 m = *(const u32x4*)(add + (size_t)idx * E + 4 * q);
#pragma unroll
        for (int e = 0; e < 4; ++e) y[4 * q + e] += as_float(m[e]);
      }
    }
    store16(o + (size_t)idx * E, Vec<T>::pack(y));
  }
}

template <typename T, int VPL>
hipError_t launch_tv(RowPass pass, const RowArgs& a, hipStream_t stream) {
  const int64_t rows = (int64_t)a.batch * a.n;
  const dim3 grid((unsigned)((rows + kWaves - 1) / kWaves)), block(64 * kWaves);
  if (pass == RowPass::kGatherNorm)
    hipLaunchKernelGGL((gather_norm_kernel<T, VPL>), grid, block, 0, stream, a);
  else if (a.addend)
    hipLaunchKernelGGL((norm_scatter_kernel<T, VPL, true>), grid, block, 0, stream, a);
  else
    hipLaunchKernelGGL((norm_scatter_kernel<T, VPL, false>), grid, block, 0, stream, a);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_t(RowPass pass, const RowArgs& a, hipStream_t stream) {
  const int per_lane = (a.channels / Vec<T>::E + 63) / 64;  // 16-byte vectors per lane
  if (per_lane <= 1) return launch_tv<T, 1>(pass, a, stream);
  if (per_lane <= 2) return launch_tv<T, 2>(pass, a, stream);
  if (per_lane <= 3) return launch_tv<T, 3>(pass, a, stream);
  if (per_lane <= 4) return launch_tv<T, 4>(pass, a, stream);
  if (per_lane <= 8) return launch_tv<T, 8>(pass, a, stream);
  if (per_lane <= 16) return launch_tv<T, 16>(pass, a, stream);
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_rows(RowPass pass, int dtype, const RowArgs& a, hipStream_t stream) {
  if ((int64_t)a.batch * a.n == 0) return hipSuccess;
  return dtype == FWN_F32 ? launch_t<float>(pass, a, stream) : launch_t<uint16_t>(pass, a, stream);
}

}  // namespace fwn
