"""MI355X-native block-sparse masked mesh attention for WeatherNext 2.

    import faster_weathernext_amd as fwn
    fwn.enable()                                    # options as the reference's enable()
    tiles = fwn.TileList.from_mask(mask)            # k-hop mask -> 128x128 live tiles (once)
    out = fwn.tiled_flash_attention(q, k, v, tiles, scale=q.shape[-1] ** -0.5)

Drop-in for the attention hot path of Raymondlol/Faster-WeatherNext (``pallas_attn.py``): the same
op contract, computed by hand-written gfx950 HIP kernels behind a C ABI (include/fwn_attn.h).
"""

from . import patch
from .hip_attn import (BLOCK_K, BLOCK_Q, TileList, attention_backward, attention_forward, tiled_flash_attention,
                       tiled_flash_attention_qkv)
from .mesh import adjacency, build_tile_mask, hilbert_order, icosahedral_mesh, khop_mask, mesh_mask
from .mha import TiledMHA
from .rows import gather_layer_norm, layer_norm_scatter
from .transformer import MeshBlock, MeshTransformer
from .tile_cache import cached_khop_tiles, cached_tile_mask

__version__ = "0.1.0"


def enable(force: bool = False, **options):
  """Selects the HIP attention path; keyword options update ``patch.Options``.

  Mirrors ``faster_weathernext.enable`` (``__init__.py:14-30``): every field of the reference's
  Options is accepted (those for parts of the reference this library does not contain have no
  effect, see ``patch.Options``), unknown options raise TypeError, an unknown ``attention`` value
  ValueError. Unless ``force`` (the reference's switch past its
  compatibility check), the native library must load and the default device must be a gfx950
  (RuntimeError otherwise). Returns the Options.
  """
  for key in options:
    if not hasattr(patch.OPTIONS, key):
      raise TypeError(f"unknown option {key!r}; see faster_weathernext_amd.patch.Options")
  if options.get("attention", patch.OPTIONS.attention) not in ("auto", "hip"):
    raise ValueError(f"unknown attention implementation {options['attention']!r} (auto, hip)")
  if options.get("precision", patch.OPTIONS.precision) not in (None,) + patch.PRECISIONS:
    raise ValueError(f"unknown precision {options['precision']!r} (None, native, bf16x3)")
  if not force:
    from . import _native
    _native.lib()
  for key, value in options.items():
    setattr(patch.OPTIONS, key, value)
  if not force:
    try:
      patch.attention_impl()
    except RuntimeError:
      patch.OPTIONS = patch.Options()
      raise
  patch.install()
  return patch.OPTIONS


def disable():
  """Restores the default options."""
  patch.uninstall()
  patch.OPTIONS = patch.Options()


def options():
  return patch.OPTIONS
