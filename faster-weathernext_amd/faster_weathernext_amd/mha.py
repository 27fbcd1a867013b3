"""The mesh transformer's attention block on the HIP kernels, with no layout copies.

Mirrors the caller of the reference's kernel, ``tiled_mha`` (``patch.py:165-177``): q, k, v
projections of the node features, masked attention over the k-hop mesh neighbourhood with
scale key_size**-0.5, reshape to [batch, n, heads * key_size] and the ``mha_final`` projection.
In the reference each projection writes [batch, n, heads, key_size], the Pallas op transposes
them to head-major and pads them (``pallas_attn.py:334-335``), and transposes the output back
(``pallas_attn.py:354``).

Here one fused projection writes q, k, v node-major into one [batch, n, 3, heads, key_size]
buffer. The kernels read the three views where they lie and write dq, dk, dv into one packed
gradient. The output [batch, n, heads, key_size] is already the [batch, n, heads * key_size]
input of the final projection. The parameters are plain torch Linear layers initialised by
torch; official WeatherNext checkpoints are Haiku parameters of the JAX model, which this
package does not load.
"""
import torch

from .hip_attn import TileList, tiled_flash_attention, tiled_flash_attention_qkv


class TiledMHA(torch.nn.Module):
  """x [batch, n, d_model] -> x's attention update [batch, n, d_model].

  ``tiles`` is the mesh's TileList (or the array triple of ``build_tile_mask``), built once and
  shared by every layer; ``tiles_t`` is the transposed mask's list for non-symmetric masks.
  """

  def __init__(self, d_model, num_heads, key_size, tiles, tiles_t=None, *, device=None, dtype=None):
    super().__init__()
    self.num_heads, self.key_size = num_heads, key_size
    self.tiles, self.tiles_t = tiles, tiles_t
    self.qkv = torch.nn.Linear(d_model, 3 * num_heads * key_size, bias=False, device=device, dtype=dtype)
    self.final = torch.nn.Linear(num_heads * key_size, d_model, device=device, dtype=dtype)

  def forward(self, x):
    b, n, _ = x.shape
    qkv = self.qkv(x).view(b, n, 3, self.num_heads, self.key_size)
    out = tiled_flash_attention_qkv(qkv, self.tiles, scale=self.key_size ** -0.5, tiles_t=self.tiles_t)
    return self.final(out.view(b, n, self.num_heads * self.key_size))

  def forward_unfused(self, x):
    """The same block with separate q, k, v tensors copied to contiguous [batch, n, heads,
    key_size] layouts, as three separate projections would leave them (comparison path)."""
    b, n, _ = x.shape
    q, k, v = (t.contiguous() for t in self.qkv(x).view(b, n, 3, self.num_heads, self.key_size).unbind(2))
    tiles = self.tiles if isinstance(self.tiles, TileList) else tuple(self.tiles)
    if isinstance(tiles, tuple):
      out = tiled_flash_attention(q, k, v, *tiles, scale=self.key_size ** -0.5, tiles_t=self.tiles_t)
    else:
      out = tiled_flash_attention(q, k, v, tiles, scale=self.key_size ** -0.5, tiles_t=self.tiles_t)
    return self.final(out.reshape(b, n, self.num_heads * self.key_size))
