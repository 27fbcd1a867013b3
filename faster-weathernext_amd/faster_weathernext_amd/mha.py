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

from . import patch
from .hip_attn import TileList, tiled_flash_attention, tiled_flash_attention_qkv

# hipBLASLt's bf16 GEMMs on MI355X run much faster when the row count is a multiple of 512: for
# the block's four GEMMs at n = 40,962 nodes, 680 us per block against 519 us at 40,960 rows.
ROW_QUANTUM = 512


def linear_rows(x, weight, bias=None, gelu=False):
  """x [M, K] @ weight[N, K]^T (+ bias) (then tanh GELU when `gelu`), without autograd.

  Runs as two GEMMs into one output: the largest multiple of ROW_QUANTUM rows, then the rest,
  so most rows get the fast kernels (for M = 40,962: 556 us per block instead of 680). The
  bias and GELU run in the GEMM epilogue. Row results do not depend on the split beyond the
  GEMM kernels' own accumulation order.
  """
  m_all = x.shape[0]
  out = torch.empty((m_all, weight.shape[0]), device=x.device, dtype=x.dtype)
  m = m_all - m_all % ROW_QUANTUM
  for lo, hi in ((0, m), (m, m_all)) if 0 < m < m_all else ((0, m_all),):
    xs, o = x[lo:hi], out[lo:hi]
    if gelu:
      torch._addmm_activation(bias, xs, weight.t(), use_gelu=True, out=o)
    elif bias is not None:
      torch.addmm(bias, xs, weight.t(), out=o)
    else:
      torch.mm(xs, weight.t(), out=o)
  return out


def needs_grad(x, module):
  """True when autograd has to see this module's computation on x."""
  return torch.is_grad_enabled() and (x.requires_grad or any(p.requires_grad for p in module.parameters()))


class TiledMHA(torch.nn.Module):
  """x [batch, n, d_model] -> x's attention update [batch, n, d_model].

  ``tiles`` is the mesh's TileList (or the array triple of ``build_tile_mask``), built once and
  shared by every layer; ``tiles_t`` is the transposed mask's list for non-symmetric masks.
  ``dtype`` None takes the enable() option (bfloat16 when ``bf16``, else float32), ``precision``
  None the precision ``patch.resolve_precision`` picks from the enable() options ``precision``
  and ``strict_fp32`` and torch's float32 matmul precision (float32 only: "native" or "bf16x3").
  """

  def __init__(self, d_model, num_heads, key_size, tiles, tiles_t=None, *, device=None, dtype=None, precision=None):
    super().__init__()
    dtype = patch.default_dtype(dtype)
    self.precision = patch.default_precision(precision, dtype)
    self.num_heads, self.key_size = num_heads, key_size
    self.tiles, self.tiles_t = tiles, tiles_t
    self.qkv = torch.nn.Linear(d_model, 3 * num_heads * key_size, bias=False, device=device, dtype=dtype)
    self.final = torch.nn.Linear(num_heads * key_size, d_model, device=device, dtype=dtype)

  def forward(self, x):
    b, n, d = x.shape
    hd = self.num_heads * self.key_size
    if needs_grad(x, self):
      qkv = self.qkv(x).view(b, n, 3, self.num_heads, self.key_size)
      out = tiled_flash_attention_qkv(qkv, self.tiles, scale=self.key_size ** -0.5, tiles_t=self.tiles_t,
                                      precision=self.precision)
      return self.final(out.view(b, n, hd))
    # Without autograd the projections run through linear_rows (the faster GEMM row split).
    qkv = linear_rows(x.reshape(b * n, d), self.qkv.weight).view(b, n, 3, self.num_heads, self.key_size)
    out = tiled_flash_attention_qkv(qkv, self.tiles, scale=self.key_size ** -0.5, tiles_t=self.tiles_t,
                                      precision=self.precision)
    return linear_rows(out.reshape(b * n, hd), self.final.weight, self.final.bias).view(b, n, -1)

  def forward_unfused(self, x):
    """The same block with separate q, k, v tensors copied to contiguous [batch, n, heads,
    key_size] layouts, as three separate projections would leave them (comparison path)."""
    b, n, _ = x.shape
    q, k, v = (t.contiguous() for t in self.qkv(x).view(b, n, 3, self.num_heads, self.key_size).unbind(2))
    tiles = self.tiles if isinstance(self.tiles, TileList) else tuple(self.tiles)
    if isinstance(tiles, tuple):
      out = tiled_flash_attention(q, k, v, *tiles, scale=self.key_size ** -0.5, tiles_t=self.tiles_t,
                                  precision=self.precision)
    else:
      out = tiled_flash_attention(q, k, v, tiles, scale=self.key_size ** -0.5, tiles_t=self.tiles_t,
                                  precision=self.precision)
    return self.final(out.reshape(b, n, self.num_heads * self.key_size))
