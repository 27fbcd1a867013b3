// C ABI: argument validation, error reporting and kernel launches.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>

#include "attn_kernels.h"
#include "fwn_attn.h"
#include "fwn_internal.h"

namespace fwn {
namespace {
thread_local char g_error[512] = "";
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_error[0] = '\0'; }

int check_tile_list(int32_t n_blocks, int32_t n_tiles, int32_t n_cols, const int32_t* ptr,
                    const int32_t* col) {
  if (ptr[0] != 0) return fail(FWN_ERR_TILES, "tile list: ptr[0] = %d, expected 0", ptr[0]);
  const int32_t n_kb = (n_cols + FWN_BLOCK - 1) / FWN_BLOCK;
  for (int32_t b = 0; b < n_blocks; ++b) {
    if (ptr[b + 1] < ptr[b]) return fail(FWN_ERR_TILES, "tile list: ptr decreases at block %d", b);
    for (int32_t t = ptr[b]; t < ptr[b + 1] && t < n_tiles; ++t) {
      if (col[t] < 0 || col[t] >= n_kb)
        return fail(FWN_ERR_TILES, "tile list: tile %d column block %d outside [0, %d)", t, col[t], n_kb);
      if (t > ptr[b] && col[t] <= col[t - 1])
        return fail(FWN_ERR_TILES, "tile list: column blocks of block %d not strictly increasing", b);
    }
  }
  if (ptr[n_blocks] != n_tiles)
    return fail(FWN_ERR_TILES, "tile list: ptr[n_blocks] = %d, expected n_tiles = %d", ptr[n_blocks], n_tiles);
  return FWN_OK;
}

namespace {

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int check_desc(const fwn_attn_desc* d) {
  if (!d) return fail(FWN_ERR_INVALID_ARG, "null descriptor");
  if (d->batch <= 0 || d->n <= 0 || d->heads <= 0)
    return fail(FWN_ERR_INVALID_ARG, "batch, n and heads must be positive (got %d, %d, %d)", d->batch, d->n,
                d->heads);
  if (d->head_dim != 32 && d->head_dim != 64 && d->head_dim != 128)
    return fail(FWN_ERR_UNSUPPORTED, "head_dim %d not built (32, 64, 128)", d->head_dim);
  if (d->dtype != FWN_F32 && d->dtype != FWN_BF16)
    return fail(FWN_ERR_UNSUPPORTED, "dtype %d not supported (0 = f32, 1 = bf16)", d->dtype);
  if (!(d->scale > 0.f) || !std::isfinite(d->scale))
    return fail(FWN_ERR_INVALID_ARG, "scale must be positive and finite");
  if (d->precision != FWN_PREC_NATIVE && d->precision != FWN_PREC_BF16X3)
    return fail(FWN_ERR_UNSUPPORTED, "precision %d not supported (0 = native, 1 = bf16x3)", d->precision);
  if (d->precision == FWN_PREC_BF16X3) {
    if (d->dtype != FWN_F32) return fail(FWN_ERR_UNSUPPORTED, "bf16x3 precision needs float32 tensors");
    // The split k and v slices are n rows of 4 * head_dim bytes, addressed with 32-bit offsets,
    // and the split pass indexes 8-element chunks with 32-bit integers.
    if ((int64_t)d->n * 4 * d->head_dim >= ((int64_t)1 << 31) ||
        (int64_t)d->batch * d->heads * d->n * (d->head_dim / 8) >= ((int64_t)1 << 31))
      return fail(FWN_ERR_INVALID_ARG, "bf16x3: batch * heads * n too large for the split pass");
  }
  const int64_t vec = d->dtype == FWN_BF16 ? 8 : 4;  // elements per 16 bytes
  const int64_t n_blocks = (d->n + FWN_BLOCK - 1) / FWN_BLOCK;
  if (n_blocks * d->batch * d->heads > INT32_MAX)
    return fail(FWN_ERR_INVALID_ARG, "grid too large");
  const int64_t elem = d->dtype == FWN_BF16 ? 2 : 4;
  const bool same = d->ostride_b == 0 && d->ostride_n == 0 && d->ostride_h == 0;
  for (int set = 0; set < (same ? 1 : 2); ++set) {
    const int64_t sb = set ? d->ostride_b : d->stride_b, sn = set ? d->ostride_n : d->stride_n,
                  sh = set ? d->ostride_h : d->stride_h;
    const char* what = set ? "o/dout strides" : "strides";
    if (sb < 0 || sn <= 0 || sh < 0 || sb % vec || sn % vec || sh % vec)
      return fail(FWN_ERR_INVALID_ARG, "%s must be non-negative multiples of 16 bytes", what);
    if (sn < d->head_dim || (d->heads > 1 && sh < d->head_dim))
      return fail(FWN_ERR_INVALID_ARG, "%s overlap rows or heads", what);
    // Buffer offsets are 32-bit: every row of a (batch, head) slice, padding rows of the last
    // block included, must be addressable below 2 GiB.
    if ((n_blocks * FWN_BLOCK + 1) * sn * elem >= ((int64_t)1 << 31))
      return fail(FWN_ERR_INVALID_ARG, "a (batch, head) slice spans 2 GiB or more (%s)", what);
  }
  return FWN_OK;
}

// Outputs are written through one of the two stride sets (o through the o set; dq, dk, dv through
// the q set), so their (batch, row, head) rows of head_dim elements must not overlap, or two work
// items would race on the same memory. Sufficient test: with the dimensions of size > 1 sorted by
// stride, each stride reaches past the extent of the ones before it.
int check_disjoint(const fwn_attn_desc* d, bool o_set, const char* what) {
  const bool same = d->ostride_b == 0 && d->ostride_n == 0 && d->ostride_h == 0;
  const bool use_o = o_set && !same;
  int64_t st[3] = {use_o ? d->ostride_b : d->stride_b, use_o ? d->ostride_n : d->stride_n,
                   use_o ? d->ostride_h : d->stride_h};
  int64_t sz[3] = {d->batch, d->n, d->heads};
  // insertion sort of the three (stride, size) pairs by stride
  for (int a = 1; a < 3; ++a)
    for (int b = a; b > 0 && st[b] < st[b - 1]; --b) {
      const int64_t t = st[b]; st[b] = st[b - 1]; st[b - 1] = t;
      const int64_t u = sz[b]; sz[b] = sz[b - 1]; sz[b - 1] = u;
    }
  int64_t extent = d->head_dim;
  for (int a = 0; a < 3; ++a) {
    if (sz[a] <= 1) continue;
    if (st[a] < extent)
      return fail(FWN_ERR_INVALID_ARG, "%s: the (batch, row, head) rows of the strides overlap", what);
    extent = st[a] * (sz[a] - 1) + extent;
  }
  return FWN_OK;
}

int check_tensor(const void* p, const char* name) {
  if (!p) return fail(FWN_ERR_INVALID_ARG, "%s is null", name);
  if (!aligned16(p)) return fail(FWN_ERR_INVALID_ARG, "%s is not 16-byte aligned", name);
  return FWN_OK;
}

int check_tiles(const fwn_attn_desc* d, const fwn_tiles* t, const char* name) {
  if (!t) return fail(FWN_ERR_INVALID_ARG, "%s is null", name);
  const int32_t n_blocks = (d->n + FWN_BLOCK - 1) / FWN_BLOCK;
  if (t->n_blocks != n_blocks)
    return fail(FWN_ERR_TILES, "%s has %d row blocks, expected %d for n = %d", name, t->n_blocks, n_blocks, d->n);
  if (t->n_tiles < 0 || !t->ptr || (t->n_tiles > 0 && (!t->col || !t->lanes || !t->groups)))
    return fail(FWN_ERR_TILES, "%s: missing device arrays", name);
  if (t->n_items < n_blocks || !t->items)
    return fail(FWN_ERR_TILES, "%s: %d work items for %d blocks (every block needs at least one)", name, t->n_items,
                n_blocks);
  if (t->n_parts < 0 || t->n_split < 0 || (t->n_split > 0 && !t->split) || (t->n_split > 0) != (t->n_parts > 0))
    return fail(FWN_ERR_TILES, "%s: inconsistent split schedule (%d parts, %d split blocks)", name, t->n_parts,
                t->n_split);
  if (t->work) {
    // An order table serves the (batch, head) count it was built for and holds every job.
    if (t->work_pairs != d->batch * d->heads)
      return fail(FWN_ERR_TILES, "%s: order table built for %d (batch, head) pairs, the call has %d", name,
                  t->work_pairs, d->batch * d->heads);
    if ((int64_t)t->n_work < (int64_t)t->n_items * d->batch * d->heads)
      return fail(FWN_ERR_TILES, "%s: order table of %d entries for %lld jobs", name, t->n_work,
                  (long long)t->n_items * d->batch * d->heads);
  } else if (t->n_work != 0) {
    return fail(FWN_ERR_TILES, "%s: %d order table entries but no table", name, t->n_work);
  }
  if ((int64_t)t->n_items * d->batch * d->heads > INT32_MAX ||
      (int64_t)t->n_split * d->batch * d->heads * (d->head_dim / 16) > INT32_MAX)
    return fail(FWN_ERR_INVALID_ARG, "%s: grid too large", name);
  return FWN_OK;
}

uint64_t partial_bytes(const fwn_attn_desc* d, const fwn_tiles* t) {
  return (uint64_t)t->n_parts * (uint64_t)d->batch * (uint64_t)d->heads * (uint64_t)slot_words(d->head_dim) * 4u;
}

// Bytes of one split tensor (bf16x3 forward): batch * heads * n rows of hi and lo bf16.
uint64_t split_bytes(const fwn_attn_desc* d) {
  return (uint64_t)d->batch * (uint64_t)d->heads * (uint64_t)d->n * (uint64_t)d->head_dim * 4u;
}

uint64_t round256(uint64_t x) { return (x + 255u) & ~(uint64_t)255u; }

// Partial slots, then (bf16x3) three split tensors, each from a 256-byte boundary: the forward
// splits k and v into slots 0 and 1, dK/dV q and dout into 0 and 1, dQ k into 2.
uint64_t workspace_bytes_for(const fwn_attn_desc* d, const fwn_tiles* t) {
  const uint64_t parts = partial_bytes(d, t);
  if (d->precision != FWN_PREC_BF16X3) return parts;
  return round256(parts) + 3u * round256(split_bytes(d));
}

// Splits the float32 tensor x (strides sb, sn, sh) into split slot `slot` of the workspace (stream
// order); returns the slot's address in *out.
int split_to_slot(const fwn_attn_desc* d, const fwn_tiles* t, void* ws, int slot, const void* x, int64_t sb,
                  int64_t sn, int64_t sh, hipStream_t stream, const uint16_t** out) {
  uint16_t* dst = (uint16_t*)((char*)ws + round256(partial_bytes(d, t)) + (uint64_t)slot * round256(split_bytes(d)));
  if (hipError_t e = launch_split_x3((const float*)x, sb, sn, sh, d->batch, d->n, d->heads, d->head_dim, dst, stream);
      e != hipSuccess)
    return fail(FWN_ERR_HIP, "bf16x3 split launch: %s", hipGetErrorString(e));
  *out = dst;
  return FWN_OK;
}

// The backward kernels compute in the tensors' dtype only.
int check_native(const fwn_attn_desc* d, const char* what) {
  if (d->precision != FWN_PREC_NATIVE)
    return fail(FWN_ERR_UNSUPPORTED, "%s: only FWN_PREC_NATIVE is built (got precision %d)", what, d->precision);
  return FWN_OK;
}

int check_workspace(const fwn_attn_desc* d, const fwn_tiles* t, const void* ws, uint64_t ws_bytes) {
  const uint64_t need = workspace_bytes_for(d, t);
  if (need == 0) return FWN_OK;
  if (!ws) return fail(FWN_ERR_INVALID_ARG, "workspace is null but %llu bytes are needed", (unsigned long long)need);
  if (((uintptr_t)ws & 255u) != 0) return fail(FWN_ERR_INVALID_ARG, "workspace is not 256-byte aligned");
  if (ws_bytes < need)
    return fail(FWN_ERR_INVALID_ARG, "workspace holds %llu bytes, %llu needed", (unsigned long long)ws_bytes,
                (unsigned long long)need);
  return FWN_OK;
}

KArgs base_args(const fwn_attn_desc* d) {
  KArgs a = {};
  a.n = d->n;
  a.heads = d->heads;
  a.batch = d->batch;
  a.n_blocks = (d->n + FWN_BLOCK - 1) / FWN_BLOCK;
  a.sb = d->stride_b;
  a.sn = d->stride_n;
  a.sh = d->stride_h;
  const bool same = d->ostride_b == 0 && d->ostride_n == 0 && d->ostride_h == 0;
  a.osb = same ? d->stride_b : d->ostride_b;
  a.osn = same ? d->stride_n : d->ostride_n;
  a.osh = same ? d->stride_h : d->ostride_h;
  const int64_t elem = d->dtype == FWN_BF16 ? 2 : 4;
  a.slice_bytes = (uint32_t)(((int64_t)(d->n - 1) * a.sn + d->head_dim) * elem);
  a.oslice_bytes = (uint32_t)(((int64_t)(d->n - 1) * a.osn + d->head_dim) * elem);
  a.scale = d->scale;
  a.c2 = (float)((double)d->scale * 1.4426950408889634);
  a.nlse_mul = (float)(-1.0 / (double)d->scale);
  return a;
}

void set_tiles(KArgs& a, const fwn_tiles* t, void* ws) {
  a.ptr = t->ptr;
  a.col = t->col;
  a.lanes = t->lanes;
  a.groups = t->groups;
  a.halves = t->halves;
  a.items = (const int32_t*)t->items;
  a.split = t->split;
  a.n_tiles = t->n_tiles;
  a.n_items = t->n_items;
  a.n_parts = t->n_parts;
  a.n_split = t->n_split;
  a.order = t->work;
  a.n_order = t->work ? t->n_work : 0;
  a.work = (float*)ws;
}

// The main kernel, then (when the list has split blocks) the combine pass, in stream order.
int launch_with_combine(Kind kind, Kind combine, const fwn_attn_desc* d, const KArgs& a, hipStream_t stream,
                        const char* what) {
  const hipError_t err = d->precision == FWN_PREC_BF16X3 ? launch_x3(kind, d->head_dim, a, stream)
                                                          : launch(kind, d->dtype, d->head_dim, a, stream);
  if (hipError_t e = err; e != hipSuccess)
    return fail(FWN_ERR_HIP, "%s launch: %s", what, hipGetErrorString(e));
  if (a.n_split > 0) {
    if (hipError_t e = launch(combine, d->dtype, d->head_dim, a, stream); e != hipSuccess)
      return fail(FWN_ERR_HIP, "%s combine launch: %s", what, hipGetErrorString(e));
  }
  return FWN_OK;
}

// Bytes of one dS unit: 32 queries x 16 keys of bf16, or 32 x 32 of float32.
int64_t ds_unit_bytes(const fwn_ds_map* m) { return m->unit_keys == 16 ? 1024 : 4096; }

// The dS exchange needs a map and buffer that match the call: the unit size of the dtype (16
// keys for bf16, 32 for float32), n_units from fwn_tiles_ds_map, one (batch, head) slice of
// units addressable with 32-bit offsets, and ds_bytes >= batch * heads * n_units * unit bytes.
int check_ds(const fwn_attn_desc* d, const fwn_ds_map* m, const void* ds, uint64_t ds_bytes, bool need_ubase,
             bool need_tmap) {
  if (!m) return fail(FWN_ERR_INVALID_ARG, "ds map is null");
  const int32_t want = d->dtype == FWN_BF16 ? 16 : 32;
  if (m->unit_keys != want)
    return fail(FWN_ERR_INVALID_ARG, "ds map: unit_keys %d, the %s exchange uses %d", m->unit_keys,
                d->dtype == FWN_BF16 ? "bf16" : "float32", want);
  if (m->n_units < 0 || m->n_units * ds_unit_bytes(m) >= ((int64_t)1 << 31))
    return fail(FWN_ERR_INVALID_ARG, "ds map: %lld units of %lld bytes (a (batch, head) slice must stay below 2 GiB)",
                (long long)m->n_units, (long long)ds_unit_bytes(m));
  // Every listed tile holds a valid element, hence a unit: a map without units belongs to lists
  // without tiles, whose per-tile arrays are empty and may be null.
  if (m->n_units > 0 && ((need_ubase && !m->ubase) || (need_tmap && !m->tmap)))
    return fail(FWN_ERR_INVALID_ARG, "ds map: null arrays");
  if (!ds) return fail(FWN_ERR_INVALID_ARG, "ds is null");
  if (((uintptr_t)ds & 255u) != 0) return fail(FWN_ERR_INVALID_ARG, "ds is not 256-byte aligned");
  const uint64_t need = (uint64_t)d->batch * (uint64_t)d->heads * (uint64_t)(m->n_units * ds_unit_bytes(m));
  if (ds_bytes < need)
    return fail(FWN_ERR_INVALID_ARG, "ds holds %llu bytes, %llu needed", (unsigned long long)ds_bytes,
                (unsigned long long)need);
  return FWN_OK;
}

void set_ds(KArgs& a, const fwn_ds_map* m, const void* ds) {
  a.ds = (uint16_t*)ds;
  a.ubase = m->ubase;
  a.tmap = m->tmap;
  a.ds_slice_bytes = (uint32_t)(m->n_units * ds_unit_bytes(m));
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return FWN_OK;
  return fail(FWN_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

}  // namespace
}  // namespace fwn

using namespace fwn;

extern "C" {

const char* fwn_last_error(void) { return fwn::g_error; }

int fwn_attn_workspace_size(const fwn_attn_desc* desc, const fwn_tiles* tiles, uint64_t* bytes) {
  clear_error();
  if (int rc = check_desc(desc)) return rc;
  if (int rc = check_tiles(desc, tiles, "tiles")) return rc;
  if (!bytes) return fail(FWN_ERR_INVALID_ARG, "bytes is null");
  *bytes = workspace_bytes_for(desc, tiles);
  return FWN_OK;
}

int fwn_attn_fwd_launch(const fwn_attn_desc* desc, const void* q, const void* k, const void* v,
                        const fwn_tiles* tiles, void* o, float* lse, void* workspace, uint64_t workspace_bytes,
                        void* stream) {
  clear_error();
  if (int rc = check_desc(desc)) return rc;
  if (int rc = check_tensor(q, "q")) return rc;
  if (int rc = check_tensor(k, "k")) return rc;
  if (int rc = check_tensor(v, "v")) return rc;
  if (int rc = check_tensor(o, "o")) return rc;
  if (int rc = check_disjoint(desc, true, "o")) return rc;
  if (int rc = check_tiles(desc, tiles, "tiles")) return rc;
  if (int rc = check_workspace(desc, tiles, workspace, workspace_bytes)) return rc;
  KArgs a = base_args(desc);
  a.q = q;
  a.k = k;
  a.v = v;
  a.out0 = o;
  a.lse_out = lse;
  set_tiles(a, tiles, workspace);
  if (desc->precision == FWN_PREC_BF16X3) {
    // k and v split into the workspace after the partial slots, in stream order before the forward.
    const hipStream_t st = (hipStream_t)stream;
    if (int rc = split_to_slot(desc, tiles, workspace, 0, k, a.sb, a.sn, a.sh, st, &a.xa)) return rc;
    if (int rc = split_to_slot(desc, tiles, workspace, 1, v, a.sb, a.sn, a.sh, st, &a.xb)) return rc;
    a.xslice_bytes = (uint32_t)((int64_t)desc->n * 4 * desc->head_dim);
  }
  return launch_with_combine(Kind::kFwd, Kind::kFwdCombine, desc, a, (hipStream_t)stream, "forward");
}

int fwn_attn_bwd_delta_launch(const fwn_attn_desc* desc, const void* o, const void* dout, float* delta,
                              void* stream) {
  clear_error();
  if (int rc = check_desc(desc)) return rc;
  if (int rc = check_tensor(o, "o")) return rc;
  if (int rc = check_tensor(dout, "dout")) return rc;
  if (!delta) return fail(FWN_ERR_INVALID_ARG, "delta is null");
  // The delta kernel's grid: one workgroup per 8 rows (float32, head_dim 128; more rows otherwise)
  // of each batch member, in one 32-bit grid dimension.
  if (((int64_t)desc->n + 7) / 8 * desc->batch > INT32_MAX)
    return fail(FWN_ERR_INVALID_ARG, "delta: batch * n too large for one launch (%d x %d)", desc->batch, desc->n);
  KArgs a = base_args(desc);
  a.o = o;
  a.dout = dout;
  a.lse_out = delta;
  return hip_status(launch(Kind::kDelta, desc->dtype, desc->head_dim, a, (hipStream_t)stream), "delta launch");
}

int fwn_attn_bwd_dq_launch(const fwn_attn_desc* desc, const void* q, const void* k, const void* v,
                           const void* dout, const float* lse, const float* delta, const fwn_tiles* tiles,
                           void* dq, void* workspace, uint64_t workspace_bytes, void* stream) {
  clear_error();
  if (int rc = check_desc(desc)) return rc;
  if (int rc = check_native(desc, "bwd_dq")) return rc;
  if (int rc = check_tensor(q, "q")) return rc;
  if (int rc = check_tensor(k, "k")) return rc;
  if (int rc = check_tensor(v, "v")) return rc;
  if (int rc = check_tensor(dout, "dout")) return rc;
  if (int rc = check_tensor(dq, "dq")) return rc;
  if (int rc = check_disjoint(desc, false, "dq")) return rc;
  if (!lse || !delta) return fail(FWN_ERR_INVALID_ARG, "lse and delta are required");
  if (int rc = check_tiles(desc, tiles, "tiles")) return rc;
  if (int rc = check_workspace(desc, tiles, workspace, workspace_bytes)) return rc;
  KArgs a = base_args(desc);
  a.q = q;
  a.k = k;
  a.v = v;
  a.dout = dout;
  a.lse = lse;
  a.delta = delta;
  a.out0 = dq;
  set_tiles(a, tiles, workspace);
  return launch_with_combine(Kind::kDq, Kind::kDqCombine, desc, a, (hipStream_t)stream, "dq");
}

int fwn_attn_bwd_dkv_launch(const fwn_attn_desc* desc, const void* q, const void* k, const void* v,
                            const void* dout, const float* lse, const float* delta, const fwn_tiles* tiles_t,
                            void* dk, void* dv, void* workspace, uint64_t workspace_bytes, void* stream) {
  clear_error();
  if (int rc = check_desc(desc)) return rc;
  if (int rc = check_native(desc, "bwd_dkv")) return rc;
  if (int rc = check_tensor(q, "q")) return rc;
  if (int rc = check_tensor(k, "k")) return rc;
  if (int rc = check_tensor(v, "v")) return rc;
  if (int rc = check_tensor(dout, "dout")) return rc;
  if (int rc = check_tensor(dk, "dk")) return rc;
  if (int rc = check_tensor(dv, "dv")) return rc;
  if (int rc = check_disjoint(desc, false, "dk/dv")) return rc;
  if (!lse || !delta) return fail(FWN_ERR_INVALID_ARG, "lse and delta are required");
  if (int rc = check_tiles(desc, tiles_t, "tiles_t")) return rc;
  if (int rc = check_workspace(desc, tiles_t, workspace, workspace_bytes)) return rc;
  KArgs a = base_args(desc);
  a.q = q;
  a.k = k;
  a.v = v;
  a.dout = dout;
  a.lse = lse;
  a.delta = delta;
  a.out0 = dk;
  a.out1 = dv;
  set_tiles(a, tiles_t, workspace);
  return launch_with_combine(Kind::kDkv, Kind::kDkvCombine, desc, a, (hipStream_t)stream, "dkv");
}

int fwn_attn_bwd_launch(const fwn_attn_desc* desc, const void* q, const void* k, const void* v, const void* o,
                        const void* dout, const float* lse, float* delta, const fwn_tiles* tiles,
                        const fwn_tiles* tiles_t, void* dq, void* dk, void* dv, void* workspace,
                        uint64_t workspace_bytes, void* stream) {
  if (int rc = fwn_attn_bwd_delta_launch(desc, o, dout, delta, stream)) return rc;
  if (int rc = fwn_attn_bwd_dq_launch(desc, q, k, v, dout, lse, delta, tiles, dq, workspace, workspace_bytes, stream))
    return rc;
  return fwn_attn_bwd_dkv_launch(desc, q, k, v, dout, lse, delta, tiles_t ? tiles_t : tiles, dk, dv, workspace,
                                 workspace_bytes, stream);
}

int fwn_attn_ds_bytes(const fwn_attn_desc* desc, const fwn_ds_map* map, uint64_t* bytes) {
  clear_error();
  if (int rc = check_desc(desc)) return rc;
  if (!map || !bytes) return fail(FWN_ERR_INVALID_ARG, "map and bytes are required");
  if (map->n_units < 0) return fail(FWN_ERR_INVALID_ARG, "ds map: negative unit count");
  if (map->unit_keys != 16 && map->unit_keys != 32)
    return fail(FWN_ERR_INVALID_ARG, "ds map: unit_keys %d (16 or 32)", map->unit_keys);
  *bytes = (uint64_t)desc->batch * (uint64_t)desc->heads * (uint64_t)(map->n_units * ds_unit_bytes(map));
  return FWN_OK;
}

int fwn_attn_bwd_dkv_ds_launch(const fwn_attn_desc* desc, const void* q, const void* k, const void* v,
                               const void* dout, const float* lse, const float* delta, const fwn_tiles* tiles_t,
                               const fwn_ds_map* map, void* dk, void* dv, void* ds, uint64_t ds_bytes,
                               void* workspace, uint64_t workspace_bytes, void* stream) {
  clear_error();
  if (int rc = check_desc(desc)) return rc;
  if (int rc = check_ds(desc, map, ds, ds_bytes, false, true)) return rc;
  if (int rc = check_tensor(q, "q")) return rc;
  if (int rc = check_tensor(k, "k")) return rc;
  if (int rc = check_tensor(v, "v")) return rc;
  if (int rc = check_tensor(dout, "dout")) return rc;
  if (int rc = check_tensor(dk, "dk")) return rc;
  if (int rc = check_tensor(dv, "dv")) return rc;
  if (int rc = check_disjoint(desc, false, "dk/dv")) return rc;
  if (!lse || !delta) return fail(FWN_ERR_INVALID_ARG, "lse and delta are required");
  if (int rc = check_tiles(desc, tiles_t, "tiles_t")) return rc;
  if (int rc = check_workspace(desc, tiles_t, workspace, workspace_bytes)) return rc;
  KArgs a = base_args(desc);
  a.q = q;
  a.k = k;
  a.v = v;
  a.dout = dout;
  a.lse = lse;
  a.delta = delta;
  a.out0 = dk;
  a.out1 = dv;
  set_tiles(a, tiles_t, workspace);
  set_ds(a, map, ds);
  if (desc->precision == FWN_PREC_BF16X3) {
    const hipStream_t st = (hipStream_t)stream;
    if (int rc = split_to_slot(desc, tiles_t, workspace, 0, q, a.sb, a.sn, a.sh, st, &a.xa)) return rc;
    if (int rc = split_to_slot(desc, tiles_t, workspace, 1, dout, a.osb, a.osn, a.osh, st, &a.xb)) return rc;
    a.xslice_bytes = (uint32_t)((int64_t)desc->n * 4 * desc->head_dim);
  }
  return launch_with_combine(Kind::kDkvDs, Kind::kDkvCombine, desc, a, (hipStream_t)stream, "dkv (dS exchange)");
}

int fwn_attn_bwd_dq_ds_launch(const fwn_attn_desc* desc, const void* k, const void* ds, uint64_t ds_bytes,
                              const fwn_tiles* tiles, const fwn_ds_map* map, void* dq, void* workspace,
                              uint64_t workspace_bytes, void* stream) {
  clear_error();
  if (int rc = check_desc(desc)) return rc;
  if (int rc = check_ds(desc, map, ds, ds_bytes, true, false)) return rc;
  if (int rc = check_tensor(k, "k")) return rc;
  if (int rc = check_tensor(dq, "dq")) return rc;
  if (int rc = check_disjoint(desc, false, "dq")) return rc;
  if (int rc = check_tiles(desc, tiles, "tiles")) return rc;
  if (desc->dtype == FWN_BF16 && tiles->n_tiles > 0 && !tiles->halves)
    return fail(FWN_ERR_TILES, "tiles: the bf16 dS exchange needs the half bits (fwn_tiles_prepare with halves)");
  if (int rc = check_workspace(desc, tiles, workspace, workspace_bytes)) return rc;
  KArgs a = base_args(desc);
  a.k = k;
  a.out0 = dq;
  set_tiles(a, tiles, workspace);
  set_ds(a, map, ds);
  if (desc->precision == FWN_PREC_BF16X3) {
    if (int rc = split_to_slot(desc, tiles, workspace, 2, k, a.sb, a.sn, a.sh, (hipStream_t)stream, &a.xa)) return rc;
    a.xslice_bytes = (uint32_t)((int64_t)desc->n * 4 * desc->head_dim);
  }
  return launch_with_combine(Kind::kDqDs, Kind::kDqCombine, desc, a, (hipStream_t)stream, "dq (dS exchange)");
}

int fwn_attn_bwd_ds_launch(const fwn_attn_desc* desc, const void* q, const void* k, const void* v, const void* o,
                           const void* dout, const float* lse, float* delta, const fwn_tiles* tiles,
                           const fwn_tiles* tiles_t, const fwn_ds_map* map, void* dq, void* dk, void* dv, void* ds,
                           uint64_t ds_bytes, void* workspace, uint64_t workspace_bytes, void* stream) {
  if (int rc = fwn_attn_bwd_delta_launch(desc, o, dout, delta, stream)) return rc;
  if (int rc = fwn_attn_bwd_dkv_ds_launch(desc, q, k, v, dout, lse, delta, tiles_t ? tiles_t : tiles, map, dk, dv,
                                          ds, ds_bytes, workspace, workspace_bytes, stream))
    return rc;
  return fwn_attn_bwd_dq_ds_launch(desc, k, ds, ds_bytes, tiles, map, dq, workspace, workspace_bytes, stream);
}

}  // extern "C"
