// C ABI of the row permutation passes (fwn_rows.h): host-side validation, then one launch.
#include <cmath>
#include <cstdint>

#include <hip/hip_runtime.h>

#include "fwn_internal.h"
#include "fwn_rows.h"
#include "rows_kernels.h"

namespace fwn {
namespace {

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// perm may be NULL only when `permuted` is false (the conditioned layer norm without a scatter).
int check_rows(const fwn_rows_desc* d, const void* x, const int64_t* perm, const char* what, bool permuted = true) {
  if (!d || !x || (permuted && !perm)) return fail(FWN_ERR_INVALID_ARG, "%s: null descriptor, x or perm", what);
  if (d->batch < 0 || d->n < 0) return fail(FWN_ERR_INVALID_ARG, "%s: negative batch or n", what);
  if (d->channels <= 0 || d->channels % 8 != 0 || d->channels > FWN_ROWS_MAX_CHANNELS)
    return fail(FWN_ERR_INVALID_ARG, "%s: channels must be a positive multiple of 8 up to %d (got %d)", what,
                FWN_ROWS_MAX_CHANNELS, d->channels);
  if (d->dtype != FWN_F32 && d->dtype != FWN_BF16) return fail(FWN_ERR_UNSUPPORTED, "%s: dtype must be f32 or bf16", what);
  if (!(d->eps >= 0.f) || !std::isfinite(d->eps)) return fail(FWN_ERR_INVALID_ARG, "%s: eps must be finite and >= 0", what);
  if (!aligned16(x) || (perm && !aligned16(perm)))
    return fail(FWN_ERR_INVALID_ARG, "%s: x and perm must be 16-byte aligned", what);
  return FWN_OK;
}

// Byte extent of one [batch, n, channels] tensor.
uint64_t bytes(const fwn_rows_desc* d) {
  return (uint64_t)d->batch * (uint64_t)d->n * (uint64_t)d->channels * (d->dtype == FWN_F32 ? 4u : 2u);
}

bool overlap(const void* a, const void* b, uint64_t n) {
  const uintptr_t x = (uintptr_t)a, y = (uintptr_t)b;
  return n > 0 && x < y + n && y < x + n;
}

int status(hipError_t e, const char* what) {
  if (e == hipSuccess) return FWN_OK;
  return fail(FWN_ERR_HIP, "%s launch: %s", what, hipGetErrorString(e));
}

RowArgs base(const fwn_rows_desc* d, const void* x, const int64_t* perm) {
  RowArgs a{};
  a.x = x;
  a.perm = perm;
  a.batch = d->batch;
  a.n = d->n;
  a.channels = d->channels;
  a.eps = d->eps;
  return a;
}

}  // namespace
}  // namespace fwn

extern "C" {

int fwn_rows_gather_norm_launch(const fwn_rows_desc* d, const void* x, const int64_t* perm, void* x_out,
                                void* norm_out, void* stream) {
  using namespace fwn;
  clear_error();
  const char* what = "fwn_rows_gather_norm_launch";
  if (int rc = check_rows(d, x, perm, what)) return rc;
  if (!x_out || !aligned16(x_out) || (norm_out && !aligned16(norm_out)))
    return fail(FWN_ERR_INVALID_ARG, "%s: x_out (and norm_out) must be non-null and 16-byte aligned", what);
  const uint64_t nb = bytes(d);
  if (overlap(x, x_out, nb) || (norm_out && (overlap(x, norm_out, nb) || overlap(x_out, norm_out, nb))))
    return fail(FWN_ERR_INVALID_ARG, "%s: x, x_out and norm_out must not overlap", what);
  RowArgs a = base(d, x, perm);
  a.x_out = x_out;
  a.norm_out = norm_out;
  return status(launch_rows(RowPass::kGatherNorm, d->dtype, a, (hipStream_t)stream), what);
}

int fwn_rows_norm_scatter_launch(const fwn_rows_desc* d, const void* x, const int64_t* perm, const float* mul,
                                 const float* add, void* out, void* stream) {
  using namespace fwn;
  clear_error();
  const char* what = "fwn_rows_norm_scatter_launch";
  if (int rc = check_rows(d, x, perm, what)) return rc;
  if (!out || !aligned16(out) || (mul && !aligned16(mul)) || (add && !aligned16(add)))
    return fail(FWN_ERR_INVALID_ARG, "%s: out (and mul, add) must be non-null and 16-byte aligned", what);
  if (overlap(x, out, bytes(d))) return fail(FWN_ERR_INVALID_ARG, "%s: x and out must not overlap", what);
  RowArgs a = base(d, x, perm);
  a.mul = mul;
  a.add = add;
  a.out = out;
  return status(launch_rows(RowPass::kNormScatter, d->dtype, a, (hipStream_t)stream), what);
}

int fwn_rows_norm_affine_launch(const fwn_rows_desc* d, const void* x, const float* mul, const float* add, void* out,
                                void* stream) {
  using namespace fwn;
  clear_error();
  const char* what = "fwn_rows_norm_affine_launch";
  if (int rc = check_rows(d, x, nullptr, what, false)) return rc;
  if (!out || !aligned16(out) || (mul && !aligned16(mul)) || (add && !aligned16(add)))
    return fail(FWN_ERR_INVALID_ARG, "%s: out (and mul, add) must be non-null and 16-byte aligned", what);
  if (overlap(x, out, bytes(d))) return fail(FWN_ERR_INVALID_ARG, "%s: x and out must not overlap", what);
  RowArgs a = base(d, x, nullptr);
  a.mul = mul;
  a.add = add;
  a.out = out;
  return status(launch_rows(RowPass::kNormScatter, d->dtype, a, (hipStream_t)stream), what);
}

int fwn_rows_add_norm_affine_launch(const fwn_rows_desc* d, const void* x, const void* y, const float* mul,
                                    const float* add, void* sum, void* out, void* stream) {
  using namespace fwn;
  clear_error();
  const char* what = "fwn_rows_add_norm_affine_launch";
  if (int rc = check_rows(d, x, nullptr, what, false)) return rc;
  if (!y || !sum || !out || !aligned16(y) || !aligned16(sum) || !aligned16(out) || (mul && !aligned16(mul)) ||
      (add && !aligned16(add)))
    return fail(FWN_ERR_INVALID_ARG, "%s: y, sum and out (and mul, add) must be non-null and 16-byte aligned", what);
  const uint64_t nb = bytes(d);
  if (overlap(x, out, nb) || overlap(y, out, nb) || overlap(sum, out, nb))
    return fail(FWN_ERR_INVALID_ARG, "%s: out must not overlap x, y or sum", what);
  // sum may be x or y itself (each row is read whole before its sum is written), but no other
  // overlap: a shifted alias would read rows another wave has already overwritten.
  if ((sum != x && overlap(sum, x, nb)) || (sum != y && overlap(sum, y, nb)))
    return fail(FWN_ERR_INVALID_ARG, "%s: sum must be x, y or disjoint from both", what);
  RowArgs a = base(d, x, nullptr);
  a.addend = y;
  a.x_out = sum;
  a.mul = mul;
  a.add = add;
  a.out = out;
  return status(launch_rows(RowPass::kNormScatter, d->dtype, a, (hipStream_t)stream), what);
}

}  // extern "C"
