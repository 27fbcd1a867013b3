/* fwn_rows.h - C ABI of the row permutation passes either side of the mesh transformer's layer
 * loop, fused with the layer norms next to them (same library as fwn_attn.h).
 *
 * The reference sorts the mesh nodes along a Hilbert curve so that the k-hop mask has fewer
 * live tiles: it gathers the node features with the permutation before the 24 layers and
 * scatters them back after the final norm (patch.py:274-276, 288-292). Each of those is one
 * extra pass over [batch, n, channels] per step. Here the gather is fused with the first
 * block's layer norm and the scatter with the final layer norm and its per-member affine, so
 * the permutation costs no pass of its own.
 *
 * Conventions (as in fwn_attn.h): status codes and fwn_last_error(); launchers validate on the
 * host, enqueue on `stream`, allocate nothing and keep no pointer. Tensors are contiguous
 * [batch, n, channels] in the dtype of the descriptor; statistics are computed in float32.
 * `perm` is a device array of n int64 that must be a permutation of 0..n-1. An entry outside
 * [0, n) yields a zero row (gather) or is dropped (scatter); repeated entries make the scatter
 * write one row twice in an unspecified order. Neither touches memory outside the tensors.
 */
#ifndef FWN_ROWS_H_
#define FWN_ROWS_H_

#include <stdint.h>

#include "fwn_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

#define FWN_ROWS_MAX_CHANNELS 4096

typedef struct fwn_rows_desc {
  int32_t batch;
  int32_t n;         /* rows (mesh nodes) per batch member */
  int32_t channels;  /* features per row: a multiple of 8, at most FWN_ROWS_MAX_CHANNELS */
  int32_t dtype;     /* fwn_dtype of x and of every output */
  float eps;         /* layer-norm epsilon, added to the biased variance */
} fwn_rows_desc;

/* x_out[b, i, :] = x[b, perm[i], :] and, when norm_out is not NULL,
 * norm_out[b, i, :] = (x_out[b, i, :] - mean) / sqrt(var + eps) over the channels (a layer norm
 * without scale or offset). Replaces jnp.take(node_features, perm, axis=1) before the layer
 * loop (patch.py:274-276) fused with the first block's st.layernorm(x, create_scale=False,
 * create_offset=False) (patch.py:244). x and x_out must not overlap. */
int fwn_rows_gather_norm_launch(const fwn_rows_desc* d, const void* x, const int64_t* perm,
                                void* x_out, void* norm_out, void* stream);

/* out[b, perm[i], :] = layer_norm(x[b, i, :]) * mul[b, :] + add[b, :], with mul and add float32
 * [batch, channels] (NULL means 1 and 0). Replaces the final st.layernorm, the per-member
 * affine that LinearNormConditioning applies to it (its scale and offset come from the
 * conditioning vector, computed by the caller) and jnp.take(x, argsort(perm), axis=1)
 * (patch.py:288-292). x and out must not overlap. */
int fwn_rows_norm_scatter_launch(const fwn_rows_desc* d, const void* x, const int64_t* perm,
                                 const float* mul, const float* add, void* out, void* stream);

/* out[b, i, :] = layer_norm(x[b, i, :]) * mul[b, :] + add[b, :] (mul and add float32
 * [batch, channels], NULL meaning 1 and 0): the block's conditioned layer norm in one pass, the
 * fwn_rows_norm_scatter_launch pass without a permutation. Replaces
 * norm_conditioning_layer(st.layernorm(x, create_scale=False, create_offset=False)) in front of
 * the attention and of the feed-forward of every block (patch.py:240-244, 250-251), whose
 * LinearNormConditioning scale and offset the caller evaluates from the conditioning vector.
 * x and out must not overlap. */
int fwn_rows_norm_affine_launch(const fwn_rows_desc* d, const void* x, const float* mul,
                                const float* add, void* out, void* stream);

/* sum[b, i, :] = x[b, i, :] + y[b, i, :] (added in float32, rounded once to the dtype) and
 * out[b, i, :] = layer_norm(sum[b, i, :]) * mul[b, :] + add[b, :]: the block's residual add
 * fused with the conditioned layer norm that reads its result. Replaces `x = x + mha(...)`
 * followed by the feed-forward's norm_conditioning_layer(st.layernorm(x)), and the feed-forward
 * residual followed by the next block's conditioned layer norm (patch.py:240-253). sum may be x
 * or y itself (an in-place residual update) or disjoint from both; out must not overlap x, y or
 * sum. */
int fwn_rows_add_norm_affine_launch(const fwn_rows_desc* d, const void* x, const void* y,
                                    const float* mul, const float* add, void* sum, void* out,
                                    void* stream);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif /* FWN_ROWS_H_ */
