/* fwn_attn.h - C ABI of the MI355X (gfx950) block-sparse masked mesh attention library.
 *
 * Drop-in replacement for the attention hot path of Raymondlol/Faster-WeatherNext v0.2.0
 * (src/faster_weathernext/pallas_attn.py). Plain C types only: device pointers are `void*`
 * (HIP device memory), the stream is a `hipStream_t` passed as `void*` (NULL = default stream).
 *
 * Conventions shared by every entry point:
 *   - Return 0 (FWN_OK) on success, a nonzero fwn_status on failure; fwn_last_error() then holds
 *     a thread-local message. Invalid shapes, dtypes, strides, alignments and malformed tile
 *     lists are rejected on the host before anything is launched.
 *   - Launchers enqueue work on `stream` and return without synchronising. They allocate
 *     nothing (temporary results go to a caller-provided workspace, see
 *     fwn_attn_workspace_size, or for fwn_attn_fwd_launch_noalloc to the library's static
 *     scratch), keep no pointer after returning and hold no mutable global state (beyond the
 *     per-device scratch address fwn_attn_fwd_launch_noalloc looks up on its first call), so
 *     they are re-entrant and safe under stream capture.
 *   - Tensors q, k, v, o, dout, dq, dk, dv are [batch, n, heads, head_dim] in the element strides
 *     of fwn_attn_desc (head_dim contiguous): node-major by default, read and written in place
 *     (the reference transposes to head-major and pads, pallas_attn.py:334-335; here no copy is
 *     made). q, k, v, dq, dk, dv share one set of strides, o and dout another. The stride set an
 *     output is written through (o; dq, dk, dv) must map distinct (batch, row, head) rows to
 *     disjoint memory, or the launcher returns FWN_ERR_INVALID_ARG.
 *   - lse and delta are float32 [batch, heads, n], contiguous.
 *   - Rows are processed in blocks of FWN_BLOCK = 128 and key tiles are 128 wide
 *     (the reference uses 64 x 32, pallas_attn.py:30-31).
 */
#ifndef FWN_ATTN_H_
#define FWN_ATTN_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FWN_BLOCK 128
#define FWN_WAVES 4                       /* waves per workgroup; each owns 32 rows of a block */
#define FWN_LANE_WORDS (FWN_WAVES * 64)   /* uint64 mask words per tile: one per lane of each wave */

typedef enum fwn_status {
  FWN_OK = 0,
  FWN_ERR_INVALID_ARG = 1,  /* null pointer, bad shape, stride or alignment */
  FWN_ERR_UNSUPPORTED = 2,  /* head_dim or dtype not built */
  FWN_ERR_TILES = 3,        /* malformed tile list */
  FWN_ERR_HIP = 4,          /* a HIP runtime call failed (message has hipGetErrorString) */
} fwn_status;

typedef enum fwn_dtype { FWN_F32 = 0, FWN_BF16 = 1 } fwn_dtype;

/* How the forward forms its products (the reference's dot precision, chosen in
 * pallas_attn.py:336-341 and passed to every dot):
 *   FWN_PREC_NATIVE: in the tensors' dtype: IEEE float32 products on the float32 matrix
 *     instructions (the reference's strict_fp32 F32_F32_F32) or bf16 products for bf16 tensors.
 *   FWN_PREC_BF16X3: float32 tensors only. Each operand x is split into bf16 parts
 *     hi = bf16(x), lo = bf16(x - hi) and each product is hi*hi + hi*lo + lo*hi with float32
 *     accumulation: about 16 significant bits per operand (TF32 has 11) on the bf16 matrix
 *     instructions, the role of the reference's TF32_TF32_F32_X3 under "highest". Built for
 *     the forward and the dS-exchange backward (fwn_attn_bwd_dkv_ds_launch,
 *     fwn_attn_bwd_dq_ds_launch, fwn_attn_bwd_ds_launch, with float32-sized units); each
 *     launcher first splits the tensors that stream through LDS into the workspace
 *     (fwn_attn_workspace_size counts them). The recomputing dq and dk/dv launchers return
 *     FWN_ERR_UNSUPPORTED for this mode (run them with a native descriptor).
 * A zeroed descriptor field means FWN_PREC_NATIVE. */
typedef enum fwn_precision { FWN_PREC_NATIVE = 0, FWN_PREC_BF16X3 = 1 } fwn_precision;

/* Shape of one attention call. scale multiplies q.k (the reference passes key_size**-0.5,
 * patch.py:174). Strides are in elements. stride_* apply to q, k, v and to dq, dk, dv;
 * ostride_* to o and dout, or are all 0 to mean "the same as stride_*". Two layouts let a fused
 * projection hand over q, k, v as views of one [batch, n, 3, heads, head_dim] buffer, and take
 * dq, dk, dv back in the same buffer, while o and dout stay [batch, n, heads, head_dim]. */
typedef struct fwn_attn_desc {
  int32_t batch;
  int32_t n;          /* nodes (queries = keys) */
  int32_t heads;
  int32_t head_dim;   /* 32, 64 or 128 */
  int32_t dtype;      /* fwn_dtype of q, k, v, o, dout, dq, dk, dv */
  float scale;
  int64_t stride_b;
  int64_t stride_n;
  int64_t stride_h;
  int64_t ostride_b;
  int64_t ostride_n;
  int64_t ostride_h;
  int32_t precision;  /* fwn_precision */
  int32_t reserved;   /* 0 */
} fwn_attn_desc;

/* One work item of a tile list: tiles [t0, t1) of row block `block`. With part < 0 the item
 * covers its whole block and writes the outputs directly; with part >= 0 it writes float32
 * partial results into partial slot `part` of the workspace, and a combine pass over the
 * block's slots writes the outputs (split-K: no block's tile run bounds the launch). */
typedef struct fwn_item {
  int32_t block;
  int32_t t0;
  int32_t t1;
  int32_t part;
} fwn_item;

/* Device view of a prepared tile list (see fwn_tiles_prepare, fwn_tiles_schedule_fill).
 * `ptr`/`col` are the CSR tile list of pallas_attn.build_tile_mask (pallas_attn.py:85-109) at
 * 128 x 128; `lanes` and `groups` hold its bitmasks in the kernels' layout. For the dK/dV
 * launcher the list must be the transposed mask's (rows = keys, columns = queries), as the
 * reference's tiles_t (pallas_attn.py:297-310; equal to the forward list for symmetric masks). */
typedef struct fwn_tiles {
  int32_t n_blocks;         /* row blocks: ceil(n / 128) */
  int32_t n_tiles;          /* live tiles */
  const int32_t* ptr;       /* [n_blocks + 1] */
  const int32_t* col;       /* [n_tiles] column block of each tile */
  const uint64_t* lanes;    /* [n_tiles][FWN_WAVES][64 lanes]: bit e = accumulator element e of that lane */
  const uint32_t* groups;   /* [n_tiles] bit 4r + c: rows 32r..32r+31 of the tile have a valid
                               element in columns 32c..32c+31 (the kernels skip the others);
                               bit 16 + 4r + c: every element of that 32 x 32 group is valid
                               (the kernels apply no mask there) */
  int32_t n_items;          /* work items: every block appears, empty blocks included */
  int32_t n_parts;          /* partial slots (items with part >= 0) */
  int32_t n_split;          /* blocks cut into more than one item */
  int32_t n_work;           /* entries of the order table `work`, or 0 */
  const fwn_item* items;    /* [n_items], in block order */
  const int32_t* split;     /* [n_split * 3]: block, first partial slot, slot count */
  const uint32_t* halves;   /* [n_tiles] or NULL: bit 8r + 2c + h set when rows 32r..32r+31 of the
                               tile have a valid element in columns 32c + 16h .. +15; the bf16 dq
                               kernel skips the other 16-column halves of live groups (NULL:
                               every half of a live group is processed) */
  const int32_t* work;      /* [n_work][2] or NULL: the order table (fwn_tiles_order_fill).
                               Workgroup w runs item work[2w + 1] of (batch, head) pair work[2w]
                               (pair b * heads + h), or nothing when the entry is outside the
                               call's pairs or items (padding). NULL: workgroup w runs job w of
                               the jobs in (batch, head)-major, item order, each XCD taking a
                               contiguous range of them. */
  int32_t work_pairs;       /* batch * heads the order table was built for (launches of another
                               shape are refused); the table must come from this `items` array
                               (the launchers check its size, not its entries) */
  int32_t reserved;         /* 0 */
} fwn_tiles;

/* Thread-local message of the last failure on this thread ("" if none). */
const char* fwn_last_error(void);

/* ---------------------------------------------------------------------------------------------
 * Host mask pipeline (CPU, synchronous). Replaces the trace-time numpy/scipy work of
 * patch.py:208-219: the k-hop mask (adj ** k), the Hilbert order and build_tile_mask.
 * ------------------------------------------------------------------------------------------- */

/* Number of nodes within k hops of each node (itself included) of an adjacency in CSR
 * (adj_ptr[n + 1], adj_idx; self edges optional): row i counts the nodes reachable from i in at
 * most k steps along edges i -> j, which is row i of (adj + I) ** k for directed adjacencies too.
 * Writes row_ptr[n + 1] of the k-hop mask (exclusive prefix sums). Replaces `adj ** k`
 * (patch.py:209, scripts/attn_bench.py:32). */
int fwn_khop_count(int32_t n, const int64_t* adj_ptr, const int32_t* adj_idx, int32_t k,
                   int64_t* row_ptr);

/* Fills the sorted column indices idx[row_ptr[n]] of the k-hop mask counted above. */
int fwn_khop_fill(int32_t n, const int64_t* adj_ptr, const int32_t* adj_idx, int32_t k,
                  const int64_t* row_ptr, int32_t* idx);

/* Permutation sorting points on the sphere along a 3-D Hilbert curve (Skilling's transpose
 * algorithm, `bits` bits per axis, bits <= 20), non-finite points last, ties in input order.
 * Replaces pallas_attn.hilbert_order (pallas_attn.py:41-82). */
int fwn_hilbert_order(int64_t n, const double* lat_deg, const double* lon_deg, int32_t bits,
                      int64_t* perm);

/* CSR live-tile list of a boolean mask given in CSR (row_ptr[n_rows + 1], idx), optionally
 * permuted as mask[perm][:, perm] (perm of length n_rows == n_cols, or NULL). Two passes:
 * fwn_tiles_count writes tile_ptr[ceil(n_rows / 128) + 1]; fwn_tiles_fill writes
 * tile_col[tile_ptr[last]] and tile_bits[tile_ptr[last] * 128 * 4] (bit j of word w of row r:
 * key col*128 + 32w + j); both may be NULL when the mask has no valid element (no tiles).
 * Replaces pallas_attn.build_tile_mask (pallas_attn.py:85-109). */
int fwn_tiles_count(int32_t n_rows, int32_t n_cols, const int64_t* row_ptr, const int32_t* idx,
                    const int64_t* perm, int32_t* tile_ptr);
int fwn_tiles_fill(int32_t n_rows, int32_t n_cols, const int64_t* row_ptr, const int32_t* idx,
                   const int64_t* perm, const int32_t* tile_ptr, int32_t* tile_col,
                   uint32_t* tile_bits);

/* Validates a canonical tile list (tile_ptr, tile_col, tile_bits as above, n_cols columns) and
 * converts it into the kernels' layout: lanes[n_tiles * FWN_LANE_WORDS], groups[n_tiles] and,
 * when non-NULL, halves[n_tiles] (host buffers; the caller copies them to the device). */
int fwn_tiles_prepare(int32_t n_blocks, int32_t n_tiles, int32_t n_cols, const int32_t* tile_ptr,
                      const int32_t* tile_col, const uint32_t* tile_bits, uint64_t* lanes,
                      uint32_t* groups, uint32_t* halves);

/* Work items of a tile list: the tiles of each block are cut into ceil(count / max_item_tiles)
 * runs of near-equal length (max_item_tiles <= 0 selects FWN_ITEM_TILES). The reference runs one
 * program per block (pallas_attn.py:244-247), so its launch lasts as long as its longest block;
 * splitting bounds every item. Two passes: fwn_tiles_schedule_count gives the sizes,
 * fwn_tiles_schedule_fill writes items[n_items] in block order (neighbouring blocks share most of
 * their key tiles, so running them together keeps those tiles in L2) and split[n_split * 3]
 * (host buffers). */
#define FWN_ITEM_TILES 64
int fwn_tiles_schedule_count(int32_t n_blocks, const int32_t* tile_ptr, int32_t max_item_tiles,
                             int32_t* n_items, int32_t* n_parts, int32_t* n_split);
int fwn_tiles_schedule_fill(int32_t n_blocks, const int32_t* tile_ptr, int32_t max_item_tiles,
                            fwn_item* items, int32_t* split);

/* Order table of a per-item schedule for calls of `pairs` (batch, head) pairs (no counterpart in
 * the reference, whose grid runs one program per block in block order). The GPU deals workgroups
 * round-robin over its 8 XCDs (workgroup w to XCD w mod 8), each with its own L2; each XCD then
 * starts its workgroups in id order as slots free up. The table gives each XCD a contiguous range
 * of the jobs ((batch, head)-major, then items in block order, as without a table): of equal
 * count with FWN_ORDER_ITEMS (the same jobs on the same workgroups as no table), of equal
 * estimated cost with FWN_ORDER_BALANCED. An item's cost is item_cost plus tile_cost[t] over its
 * tiles (tile_cost NULL: 1 per tile; else at least as many entries as the largest t1, none
 * negative). With window > 1 each consecutive `window` jobs of a range run longest first
 * (windows counted from the range's end, so its last `window` jobs are one window), so short
 * jobs end the launch while the jobs running together stay neighbours. FWN_ORDER_MAKESPAN starts
 * from the equal-cost ranges and moves jobs across the boundaries of the XCD that would end last
 * (its first job to the XCD before it, or its last to the one after) while that lowers the later
 * of the two ends, each end simulated as `slots` slots taking the XCD's jobs in launch order
 * (each job to the first free slot, lasting its cost): equal cost can leave one XCD with a last
 * round of a few jobs while another's ends full. `slots` is ignored by the other orders. Ranges
 * of unequal count leave padding entries (pair -1) that exit at once. fwn_tiles_order_count
 * gives n_work; fwn_tiles_order_fill writes work[n_work * 2] (host buffers). */
#define FWN_ORDER_ITEMS 0
#define FWN_ORDER_BALANCED 1
#define FWN_ORDER_MAKESPAN 2
int fwn_tiles_order_count(int32_t n_items, const fwn_item* items, const int32_t* tile_cost, int32_t item_cost,
                          int32_t pairs, int32_t order, int32_t window, int32_t slots, int32_t* n_work);
int fwn_tiles_order_fill(int32_t n_items, const fwn_item* items, const int32_t* tile_cost, int32_t item_cost,
                         int32_t pairs, int32_t order, int32_t window, int32_t slots, int32_t* work);

/* ---------------------------------------------------------------------------------------------
 * Device launchers (enqueue on `stream`).
 *
 * `workspace` is device memory of at least fwn_attn_workspace_size bytes, 256-byte aligned,
 * owned by the caller and used only between a launch and the completion of its stream work (so
 * launches on one stream may share it; launches that can overlap need their own). It may be NULL
 * when the size is 0 (no block of the tile list is split).
 * ------------------------------------------------------------------------------------------- */

/* Workspace bytes the forward, dq and dk/dv launchers need for `tiles`:
 * tiles->n_parts * batch * heads * 128 * (2 * head_dim + 2) * 4 (float32 partial outputs plus
 * the forward's per-row max and sum), rounded up to 256 bytes and, with FWN_PREC_BF16X3, plus
 * three split tensors of batch * heads * n * head_dim * 4 bytes (each rounded up to 256). */
int fwn_attn_workspace_size(const fwn_attn_desc* desc, const fwn_tiles* tiles, uint64_t* bytes);

/* Forward: o = softmax(mask(q k^T * scale)) v, walking only live tiles with an online softmax.
 * lse (natural log-sum-exp of the scaled logits per row) is written when non-NULL.
 * Replaces pallas_attn._forward/_kernel (pallas_attn.py:112-141, 235-257). */
int fwn_attn_fwd_launch(const fwn_attn_desc* desc, const void* q, const void* k, const void* v,
                        const fwn_tiles* tiles, void* o, float* lse, void* workspace,
                        uint64_t workspace_bytes, void* stream);

/* The forward launcher without a workspace argument: split work items use the library's static
 * scratch (a __device__ array of FWN_SCRATCH_BYTES that each GPU holds from the library's load
 * until the process ends), so the call allocates nothing and takes no caller memory beyond the
 * inputs and outputs. No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under graph capture, serving loops, harnesses that forbid hipMalloc).
 * Returns FWN_ERR_INVALID_ARG when the list's split schedule needs more than FWN_SCRATCH_BYTES
 * (fwn_attn_workspace_size); lists whose blocks are not split need none. The scratch's device
 * address is looked up on the first call on each device, so make that call outside graph
 * capture. Calls on one device share its scratch: calls whose kernels can overlap on one device
 * (other streams, other threads) race, so order them on one stream. FWN_PREC_NATIVE only. */
#define FWN_SCRATCH_BYTES (64ull << 20)
int fwn_attn_fwd_launch_noalloc(const fwn_attn_desc* desc, const void* q, const void* k, const void* v,
                                const fwn_tiles* tiles, void* o, float* lse, void* stream);

/* delta = rowsum(o * dout) in float32 [batch, heads, n] (pallas_attn.py:278). */
int fwn_attn_bwd_delta_launch(const fwn_attn_desc* desc, const void* o, const void* dout,
                              float* delta, void* stream);

/* dq per query block over the forward tile list, P recomputed from lse
 * (pallas_attn.py:161-184, 286-295). */
int fwn_attn_bwd_dq_launch(const fwn_attn_desc* desc, const void* q, const void* k,
                           const void* v, const void* dout, const float* lse,
                           const float* delta, const fwn_tiles* tiles, void* dq, void* workspace,
                           uint64_t workspace_bytes, void* stream);

/* dk, dv per key block over the transposed tile list; every workgroup owns its rows of dk/dv,
 * so no atomics (pallas_attn.py:187-215, 297-310). */
int fwn_attn_bwd_dkv_launch(const fwn_attn_desc* desc, const void* q, const void* k,
                            const void* v, const void* dout, const float* lse,
                            const float* delta, const fwn_tiles* tiles_t, void* dk, void* dv,
                            void* workspace, uint64_t workspace_bytes, void* stream);

/* Whole backward: delta, dq, then dk/dv, in stream order (pallas_attn._attention_bwd,
 * pallas_attn.py:274-311). delta is caller-provided scratch of [batch, heads, n] floats; the
 * workspace must hold the larger of the two lists' sizes (dq and dk/dv run one after the other
 * on `stream` and share it). The dq and dk/dv launches only read what delta and the forward
 * wrote, so a caller with two streams may instead enqueue delta, then dq and dk/dv on different
 * streams, each with its own workspace, and join them: the two kernels then fill each other's
 * idle CUs. The Python package does this only for tile lists that are not exact transposes of
 * each other; otherwise it takes the dS exchange (fwn_attn_bwd_ds_launch), which computes S and
 * dP once. */
int fwn_attn_bwd_launch(const fwn_attn_desc* desc, const void* q, const void* k, const void* v,
                        const void* o, const void* dout, const float* lse, float* delta,
                        const fwn_tiles* tiles, const fwn_tiles* tiles_t, void* dq, void* dk,
                        void* dv, void* workspace, uint64_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Backward with the dS exchange. The reference computes S and dP twice per live tile, once for
 * dQ and once for dK/dV (pallas_attn.py:172-180, 199-207). Here the dK/dV kernel also writes
 * dS = P (dP - delta) and the dQ kernel computes dQ = scale * dS K from it: 5 contractions per
 * tile instead of 7. dS is written and read in units of 32 query rows x `unit_keys` keys, one
 * per such block of a live tile with a valid element, numbered over the forward list:
 *   - bf16: unit_keys 16 (the forward list's halves bits), bf16 dS, 1 KB per unit;
 *   - float32: unit_keys 32 (its group bits 0-15), float32 dS, 4 KB per unit.
 * The two lists must be exact transposes of each other, bit for bit (fwn_tiles_ds_map checks
 * this). dQ then equals the recomputing dq kernel's up to the rounding order of S.
 * ------------------------------------------------------------------------------------------- */

/* Unit numbering of a forward tile list and its transposed list (device arrays). */
typedef struct fwn_ds_map {
  int64_t n_units;       /* units of the forward list */
  const int32_t* ubase;  /* [tiles->n_tiles] first unit of each forward tile (ubase and tmap
                            may be NULL when n_units is 0: lists without tiles) */
  const int32_t* tmap;   /* [tiles_t->n_tiles][2]: for each transposed tile, ubase and the unit
                            bits word (as int32: halves for 16, groups for 32) of the same tile of
                            the forward list */
  int32_t unit_keys;     /* 16 (bf16 calls) or 32 (float32 calls) */
  int32_t reserved;      /* 0 */
} fwn_ds_map;

/* Builds the unit numbering (host arrays) from the canonical arrays of both lists (tile_ptr,
 * tile_col, tile_bits as fwn_tiles_fill writes them, n_blocks row blocks each) for units of
 * unit_keys (16 or 32) keys: ubase[n_tiles], tmap[n_tiles_t * 2], *n_units. Returns
 * FWN_ERR_TILES when the second list is not the transpose of the first (a tile or a bit
 * differs); the recomputing backward (fwn_attn_bwd_launch) is then the one that applies. No
 * reference counterpart. */
int fwn_tiles_ds_map(int32_t n_blocks, const int32_t* tile_ptr, const int32_t* tile_col,
                     const uint32_t* tile_bits, const int32_t* tile_ptr_t, const int32_t* tile_col_t,
                     const uint32_t* tile_bits_t, int32_t unit_keys, int32_t* ubase, int32_t* tmap,
                     int64_t* n_units);

/* Bytes of the dS buffer: batch * heads * n_units * (1024 for unit_keys 16, 4096 for 32);
 * 256-byte aligned device memory. */
int fwn_attn_ds_bytes(const fwn_attn_desc* desc, const fwn_ds_map* map, uint64_t* bytes);

/* dk, dv as fwn_attn_bwd_dkv_launch, and every dS unit into `ds` (pallas_attn.py:187-215).
 * The map's unit_keys must be 16 for bf16 and 32 for float32. */
int fwn_attn_bwd_dkv_ds_launch(const fwn_attn_desc* desc, const void* q, const void* k,
                               const void* v, const void* dout, const float* lse,
                               const float* delta, const fwn_tiles* tiles_t, const fwn_ds_map* map,
                               void* dk, void* dv, void* ds, uint64_t ds_bytes, void* workspace,
                               uint64_t workspace_bytes, void* stream);

/* dq = scale * dS K over the forward list from the units fwn_attn_bwd_dkv_ds_launch wrote
 * (replaces pallas_attn._bwd_dq_kernel, pallas_attn.py:161-184, in this mode). */
int fwn_attn_bwd_dq_ds_launch(const fwn_attn_desc* desc, const void* k, const void* ds,
                              uint64_t ds_bytes, const fwn_tiles* tiles, const fwn_ds_map* map,
                              void* dq, void* workspace, uint64_t workspace_bytes, void* stream);

/* Whole backward in this mode: delta, dk/dv (+ dS), then dq, in stream order
 * (pallas_attn._attention_bwd, pallas_attn.py:274-311). `ds` holds fwn_attn_ds_bytes; the
 * workspace holds the larger of the two lists' sizes. */
int fwn_attn_bwd_ds_launch(const fwn_attn_desc* desc, const void* q, const void* k, const void* v,
                           const void* o, const void* dout, const float* lse, float* delta,
                           const fwn_tiles* tiles, const fwn_tiles* tiles_t, const fwn_ds_map* map,
                           void* dq, void* dk, void* dv, void* ds, uint64_t ds_bytes,
                           void* workspace, uint64_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FWN_ATTN_H_ */
