// Kernel argument block and launch entry points (internal, C++ only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fwn {

struct KArgs {
  const void* q;
  const void* k;
  const void* v;
  const void* o;          // forward output (delta pre-pass)
  const void* dout;
  const float* lse;       // [batch, heads, n] natural log-sum-exp (backward)
  const float* delta;     // [batch, heads, n] rowsum(o * dout) (backward)
  void* out0;             // o (fwd), dq (dq), dk (dkv)
  void* out1;             // dv (dkv)
  float* lse_out;         // fwd: optional; delta pre-pass: delta
  const int32_t* ptr;
  const int32_t* col;
  const uint64_t* lanes;
  const uint32_t* groups;  // per tile: bit 4r + c = rows 32r.. have a valid element in columns 32c..
  const uint32_t* halves;  // per tile: bit 8r + 2c + h = ... in columns 32c + 16h..; NULL = all live
  const int32_t* items;   // fwn_item[n_items] as int32 quadruples (block, t0, t1, part)
  const int32_t* split;   // [n_split * 3] block, first partial slot, slot count (combine pass)
  const int32_t* order;   // order table: [n_order][2] (pair b * heads + h, item) per workgroup, or NULL
  float* work;            // partial slots: [n_parts][batch * heads][128][2 * head_dim + 2] float32
  uint16_t* ds;           // dS units (bf16 backward with the dS exchange): [batch * heads][n_units][512]
  const int32_t* ubase;   // dq from dS: first unit of each tile of the forward list
  const int32_t* tmap;    // dK/dV writing dS: per transposed tile, (ubase, halves) of the forward tile
  uint32_t ds_slice_bytes;  // bytes of one (batch, head) slice of ds: n_units * 1024
  const uint16_t* xa;     // bf16x3 kernels: split operands, [batch * heads][n][2][head_dim] bf16 (hi row,
  const uint16_t* xb;     //   lo row; written by the split pass): forward k, v; dK/dV q, dout; dQ k
  uint32_t xslice_bytes;  // bytes of one (batch, head) slice of xa / xb: n * 4 * head_dim
  int32_t n, heads, batch, n_blocks, n_tiles, n_items, n_parts, n_split, n_order;
  int64_t sb, sn, sh;     // strides of q, k, v, dq, dk, dv
  int64_t osb, osn, osh;  // strides of o, dout
  uint32_t slice_bytes;   // bytes of one (batch, head) slice: ((n - 1) * sn + head_dim) * elem
  uint32_t oslice_bytes;  // the same for o, dout
  float scale;            // softmax scale
  float c2;               // scale * log2(e)
  float nlse_mul;         // -1 / scale: turns a saved lse into the initial value of an S accumulator
};

// kDqDs and kDkvDs: the bf16 backward with the dS exchange (dK/dV writes each 32 x 16 dS unit,
// the dQ kernel reads it instead of recomputing S and dP).
enum class Kind { kFwd, kDq, kDkv, kDelta, kFwdCombine, kDqCombine, kDkvCombine, kDqDs, kDkvDs };

// Kernel launchers (each enqueues one kernel and returns hipSuccess or the launch error).
hipError_t launch_bf16(Kind kind, int head_dim, const KArgs& a, hipStream_t stream);  // attn_bf16.hip
hipError_t launch_f32(Kind kind, int head_dim, const KArgs& a, hipStream_t stream);   // attn_f32.hip
hipError_t launch_delta_bf16(int head_dim, const KArgs& a, hipStream_t stream);      // attn_f32.hip
hipError_t launch_x3(Kind kind, int head_dim, const KArgs& a, hipStream_t stream);    // attn_x3.hip: kFwd, kDkvDs, kDqDs
// Splits a float32 [batch, n, heads, head_dim] tensor (element strides sb, sn, sh) into dst,
// [batch * heads][n][2][head_dim] bf16: hi = bf16(x), lo = bf16(x - hi) (attn_x3.hip).
hipError_t launch_split_x3(const float* src, int64_t sb, int64_t sn, int64_t sh, int batch, int n, int heads,
                           int head_dim, uint16_t* dst, hipStream_t stream);
hipError_t launch_combine(Kind kind, int dtype, int head_dim, const KArgs& a,
                          hipStream_t stream);                                     // attn_combine.hip

// Dispatch on dtype (0 f32, 1 bf16).
inline hipError_t launch(Kind kind, int dtype, int head_dim, const KArgs& a, hipStream_t stream) {
  if (kind == Kind::kFwdCombine || kind == Kind::kDqCombine || kind == Kind::kDkvCombine)
    return launch_combine(kind, dtype, head_dim, a, stream);
  if (dtype == 0) return launch_f32(kind, head_dim, a, stream);
  if (kind == Kind::kDelta) return launch_delta_bf16(head_dim, a, stream);
  return launch_bf16(kind, head_dim, a, stream);
}

// Workgroups of a per-item launch: one per entry of the order table, else one per (item, batch,
// head).
__host__ __device__ inline int64_t job_count(const KArgs& a) {
  return a.order ? (int64_t)a.n_order : (int64_t)a.n_items * a.batch * a.heads;
}

// Float32 words of one partial slot of one (batch, head): O or dQ or dK rows [128][D], then dV
// rows [128][D] (dK/dV) or the forward's row max [128] and row sum [128].
inline int64_t slot_words(int head_dim) { return 128 * (2 * (int64_t)head_dim + 2); }

}  // namespace fwn
