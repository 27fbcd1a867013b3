// Interface between the row-pass launchers (rows_api.cpp) and their kernels (rows.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fwn {

struct RowArgs {
  const void* x;
  const int64_t* perm;
  void* x_out;       // gather: permuted copy of x
  void* norm_out;    // gather: its layer norm, or null
  const float* mul;  // scatter: [batch, channels] or null
  const float* add;  // scatter: [batch, channels] or null
  void* out;         // scatter: output
  const void* addend;  // scatter: added to x before the norm (the sum goes to x_out, required then), or null
  int32_t batch, n, channels;
  float eps;
};

enum class RowPass { kGatherNorm, kNormScatter };

// Launches one pass; dtype is FWN_F32 or FWN_BF16 and channels a validated multiple of 8.
hipError_t launch_rows(RowPass pass, int dtype, const RowArgs& a, hipStream_t stream);

}  // namespace fwn
