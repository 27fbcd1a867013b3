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
  const uint32_t* full;
  const int32_t* order;
  int32_t n, heads, batch, n_blocks, n_tiles;
  int64_t sb, sn, sh;
  uint32_t slice_bytes;   // bytes of one (batch, head) slice: ((n - 1) * sn + head_dim) * elem
  float scale;            // softmax scale
  float c2;               // scale * log2(e)
};

enum class Kind { kFwd, kDq, kDkv, kDelta };

// Kernel launchers (each enqueues one kernel and returns hipSuccess or the launch error).
hipError_t launch_bf16(Kind kind, int head_dim, const KArgs& a, hipStream_t stream);  // attn_bf16.hip
hipError_t launch_f32(Kind kind, int head_dim, const KArgs& a, hipStream_t stream);   // attn_f32.hip
hipError_t launch_delta_bf16(int head_dim, const KArgs& a, hipStream_t stream);      // attn_f32.hip

// Dispatch on dtype (0 f32, 1 bf16).
inline hipError_t launch(Kind kind, int dtype, int head_dim, const KArgs& a, hipStream_t stream) {
  if (dtype == 0) return launch_f32(kind, head_dim, a, stream);
  if (kind == Kind::kDelta) return launch_delta_bf16(head_dim, a, stream);
  return launch_bf16(kind, head_dim, a, stream);
}

}  // namespace fwn
