"""The mesh transformer around the attention kernels: the reference's patched
``ChunkedTransformer`` / ``ChunkedBlock`` (``patch.py:193-293``) in PyTorch.

Structure, as the reference wires it:

* at construction, the k-hop mask of the refined icosahedral mesh, the optional Hilbert
  permutation and the live-tile list, built once and shared by every layer
  (``_transformer_init``, ``patch.py:193-226``; ``optimization_barrier``, ``:263-266``);
* before the layers, the gather of the node features into Hilbert order (``:274-276``), here
  fused with block 0's first layer norm (``rows.gather_layer_norm``);
* per block (``ChunkedBlock.__call__``, ``:233-253``):
  ``x = x + mha(cond_norm(layernorm(x)))`` then ``x = x + ffw(cond_norm(layernorm(x)))``, with the
  attention ``TiledMHA`` (``tiled_mha``, ``:165-177``) on the HIP kernels;
* after the layers, the final layer norm, its conditioning and the scatter back to mesh order
  (``:288-292``), fused into one pass (``rows.layer_norm_scatter``).

Two parts live in weathernext, which is not vendored, so their exact form is not pinned here:
``LinearNormConditioning`` is implemented as published with GenCast (a linear map of the
conditioning vector, zero-initialised, giving a per-channel scale-minus-one and offset:
``x * (1 + scale) + offset``), and ``st.ffw`` as a two-layer GELU MLP of width ``ffw_hidden``
with the tanh form of GELU (``jax.nn.gelu``'s default). Without autograd, the first layer's bias
and GELU run in the epilogue of its GEMM (``torch._addmm_activation``, which has no derivative),
so the [n, ffw_hidden] activations make one trip to HBM instead of three, every block GEMM
splits its rows at a multiple of 512 (``mha.linear_rows``), and each residual add runs in one
pass with the conditioned layer norm after it (``rows.add_layer_norm_affine``); with autograd the
same functions run as plain Linear, GELU, Linear and separate adds.
Parameters are random-initialised torch parameters; official checkpoints are Haiku parameters of
the JAX model, which this package does not load.
"""
import numpy as np
import torch
import torch.nn.functional as F
from scipy import sparse

from . import patch
from .hip_attn import TileList
from .mesh import hilbert_order, khop_mask, mesh_mask
from .mha import TiledMHA, linear_rows, needs_grad
from .rows import add_layer_norm_affine, gather_layer_norm, layer_norm_affine, layer_norm_scatter


class NormConditioning(torch.nn.Module):
  """x * (1 + scale(cond)) + offset(cond) per channel; the linear map starts at zero."""

  def __init__(self, d_model, cond_size, device=None, dtype=None):
    super().__init__()
    self.linear = torch.nn.Linear(cond_size, 2 * d_model, device=device, dtype=dtype)
    torch.nn.init.zeros_(self.linear.weight)
    torch.nn.init.zeros_(self.linear.bias)

  def affine(self, cond):
    """(multiplier, offset), each [batch, d_model]."""
    scale_m1, offset = self.linear(cond).chunk(2, dim=-1)
    return 1 + scale_m1, offset

  def forward(self, x, cond):
    mul, add = self.affine(cond)
    return x * mul[:, None, :] + add[:, None, :]

  def norm(self, x, cond, eps):
    """forward(layer_norm(x), cond) as one HIP pass (statistics and affine in float32)."""
    mul, add = self.affine(cond)
    return layer_norm_affine(x, mul=mul.float().contiguous(), add=add.float().contiguous(), eps=eps)

  def add_norm(self, x, y, cond, eps):
    """(x + y, forward(layer_norm(x + y), cond)) as one HIP pass, without autograd."""
    mul, add = self.affine(cond)
    return add_layer_norm_affine(x, y, mul=mul.float().contiguous(), add=add.float().contiguous(), eps=eps)


class MeshBlock(torch.nn.Module):
  """One transformer block (``ChunkedBlock``, ``patch.py:229-253``)."""

  def __init__(self, d_model, num_heads, key_size, ffw_hidden, cond_size, tiles, tiles_t=None, *, device=None,
               dtype=None, eps=1e-5, precision=None):
    super().__init__()
    self.eps = eps
    kw = dict(device=device, dtype=dtype)
    self.norm_mha = NormConditioning(d_model, cond_size, **kw)
    self.mha = TiledMHA(d_model, num_heads, key_size, tiles, tiles_t, precision=precision, **kw)
    self.norm_ffw = NormConditioning(d_model, cond_size, **kw)
    self.ffw = torch.nn.Sequential(torch.nn.Linear(d_model, ffw_hidden, **kw), torch.nn.GELU(approximate="tanh"),
                                   torch.nn.Linear(ffw_hidden, d_model, **kw))

  def feed_forward(self, h):
    """self.ffw(h); without autograd, the first layer's bias and GELU are fused into its GEMM and
    both GEMMs use the faster row split (``linear_rows``)."""
    l1, l2 = self.ffw[0], self.ffw[2]
    if needs_grad(h, self.ffw):
      return self.ffw(h)
    lead = h.shape[:-1]
    y = linear_rows(h.reshape(-1, h.shape[-1]), l1.weight, l1.bias, gelu=True)
    return linear_rows(y, l2.weight, l2.bias).view(*lead, l2.out_features)

  def forward(self, x, cond, normed=None):
    """`normed` is layernorm(x) when the caller has it already (block 0 gets it from the fused
    gather). Otherwise each conditioned layer norm is one fused pass (``layer_norm_affine``)."""
    h = self.norm_mha(normed, cond) if normed is not None else self.norm_mha.norm(x, cond, self.eps)
    x = x + self.mha(h)
    return x + self.feed_forward(self.norm_ffw.norm(x, cond, self.eps))

  def forward_fused(self, x, h, cond, next_norm=None):
    """The block without autograd, from h = norm_mha(layernorm(x)) already computed: each residual
    add runs in one pass with the conditioned layer norm that reads it (``add_layer_norm_affine``),
    the feed-forward's own and, when `next_norm` is given, the next block's. Returns (x, the next
    block's h or None)."""
    x, h = self.norm_ffw.add_norm(x, self.mha(h), cond, self.eps)
    f = self.feed_forward(h)
    if next_norm is None:
      return x + f, None
    return next_norm.add_norm(x, f, cond, self.eps)


class MeshTransformer(torch.nn.Module):
  """The 24-layer mesh transformer of WeatherNext 2's processor, node features [batch, n, d_model]
  in mesh (subdivision) order in and out; the attention runs in Hilbert order when `reorder`.

  The mask is the k-hop neighbourhood of the refined icosahedral mesh, or of ``adjacency`` (a
  boolean [n, n] sparse matrix, with the nodes' ``latlon`` in degrees for the Hilbert order) when
  one is given, as the reference builds it from the model's own adjacency (``patch.py:193-219``).
  A non-symmetric adjacency gives a non-symmetric mask, whose transposed tile list the backward
  walks. ``reorder``, ``dtype`` and ``precision`` None take the enable() options (``reorder``,
  ``bf16``, ``precision``).
  """

  def __init__(self, refinement=6, k_hop=32, num_layers=24, d_model=768, num_heads=6, key_size=128,
               ffw_hidden=3072, cond_size=32, reorder=None, *, device="cuda", dtype=None, tiles=None,
               tiles_t=None, adjacency=None, latlon=None, eps=1e-5, precision=None):
    super().__init__()
    reorder = patch.default_reorder(reorder)
    dtype = patch.default_dtype(dtype)
    if adjacency is None:
      mask, lat, lon, perm = mesh_mask(refinement, k_hop, reorder=reorder)
      symmetric = True  # powers of the mesh's symmetric adjacency
    else:
      adjacency = sparse.csr_matrix(adjacency).astype(bool)
      mask = khop_mask(adjacency, k_hop)
      perm = hilbert_order(*latlon) if reorder and latlon is not None else None
      symmetric = (adjacency != adjacency.T).nnz == 0
    self.n = mask.shape[0]
    self.eps = eps
    # One tile list for every layer (patch.py:214); the backward walks the transposed mask's list,
    # built only when the adjacency is not symmetric (patch.py:215-218).
    if tiles is None:
      tiles = TileList.from_mask(mask, perm, device=device)
      if not symmetric and tiles_t is None:
        permuted = mask if perm is None else mask[perm][:, perm]
        tiles_t = TileList.from_mask(permuted.T.tocsr(), device=device)
    elif not symmetric and tiles_t is None:
      # The backward would walk the forward list as its own transpose: wrong dK/dV.
      raise ValueError("a non-symmetric adjacency with caller-built tiles needs tiles_t, the transposed mask's "
                       "tile list")
    self.tiles, self.tiles_t = tiles, tiles_t
    self.register_buffer("perm", None if perm is None else torch.from_numpy(np.asarray(perm, np.int64)).to(device),
                         persistent=False)
    self.blocks = torch.nn.ModuleList(
        MeshBlock(d_model, num_heads, key_size, ffw_hidden, cond_size, self.tiles, self.tiles_t, device=device,
                  dtype=dtype, eps=eps, precision=precision)
        for _ in range(num_layers))
    self.final_norm = NormConditioning(d_model, cond_size, device=device, dtype=dtype)

  def forward(self, x, cond):
    d = x.shape[-1]
    normed = None
    if self.perm is not None:
      x, normed = gather_layer_norm(x, self.perm, eps=self.eps)
    elif len(self.blocks):
      normed = F.layer_norm(x, (d,), eps=self.eps)
    if len(self.blocks) and not needs_grad(x, self):
      # Without autograd the residual adds are fused into the conditioned layer norms after them.
      h = self.blocks[0].norm_mha(normed, cond)
      for i, block in enumerate(self.blocks):
        x, h = block.forward_fused(x, h, cond, self.blocks[i + 1].norm_mha if i + 1 < len(self.blocks) else None)
    else:
      for i, block in enumerate(self.blocks):
        x = block(x, cond, normed if i == 0 else None)
    mul, add = self.final_norm.affine(cond)
    if self.perm is not None:
      return layer_norm_scatter(x, self.perm, mul=mul.float().contiguous(), add=add.float().contiguous(), eps=self.eps)
    return F.layer_norm(x, (d,), eps=self.eps) * mul[:, None, :] + add[:, None, :]
