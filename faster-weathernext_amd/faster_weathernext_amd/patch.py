"""Execution options and the attention dispatch of the drop-in switch.

Mirrors the attention slice of the reference's ``patch.py`` (``Options`` 50-79, ``attention_impl``
86-99, ``install``/``uninstall`` 727-758). Only the options that concern the attention path are
kept; the GNN / encoder / decoder blocking options of the reference are out of scope (they exist
to fit 8-32 GB cards), and so is ``replace_attention``, which routes the official configs'
attention types inside the JAX model.

The options are read when a model is built: ``MeshTransformer`` takes its node order from
``reorder`` and, with ``TiledMHA``, its parameter and activation dtype from ``bf16`` when the
caller passes none.

The reference's patch swaps subclasses into the official ``weathernext`` modules so its
transformer calls ``pallas_attn.tiled_flash_attention``. Wiring this library into that JAX model
needs jax, haiku and weathernext plus an XLA FFI handler around the C ABI;
``missing_model_dependencies`` names what is missing here. ``install`` marks the HIP path as the
active one for the torch modules of this package.
"""
import dataclasses
import importlib.util

ARCH = "gfx950"  # the only target the kernels are built for


@dataclasses.dataclass
class Options:
  """Execution options (read when a model is built)."""
  # Attention kernel: "hip" (the gfx950 kernels of this package) or "auto" (= "hip" on gfx950).
  attention: str = "auto"
  # Process mesh nodes in Hilbert-curve order (exact; fewer live tiles). MeshTransformer's default.
  reorder: bool = True
  # bfloat16 parameters and activations with float32 accumulation instead of float32 (fp32 MFMA).
  # MeshTransformer's and TiledMHA's default dtype.
  bf16: bool = False
  # Products of the attention kernels on float32 tensors: "native" (IEEE float32 products, the
  # reference's strict_fp32) or "bf16x3" (three bf16 products per float32 product, about 16
  # significant bits per operand: the role of the reference's 3xTF32 "highest" dots, at 2.5-3.2x
  # the speed). bfloat16 tensors always take bf16 products.
  precision: str = "native"


OPTIONS = Options()
_enabled = False


def device_arch(index=0):
  """gfx target name of ROCm device `index` (e.g. "gfx950"), or None without a ROCm device."""
  import torch
  if getattr(torch.version, "hip", None) is None or not torch.cuda.is_available():
    return None
  if index >= torch.cuda.device_count():
    return None
  return torch.cuda.get_device_properties(index).gcnArchName.split(":")[0]


def attention_impl():
  """The attention implementation ``enable()`` uses: "hip", the gfx950 kernels.

  As the reference picks its kernel from the device (``patch.py:86-99``), this checks that the
  default device is a gfx950; there is no other implementation to fall back to, so any other
  device raises RuntimeError."""
  if OPTIONS.attention not in ("auto", "hip"):
    raise ValueError(f"unknown attention implementation {OPTIONS.attention!r} (auto, hip)")
  arch = device_arch()
  if arch != ARCH:
    raise RuntimeError(f"the HIP attention kernels run on {ARCH} (MI355X) only; the default device is "
                       f"{arch or 'not a ROCm GPU'}")
  return "hip"


def default_dtype(dtype=None):
  """`dtype` if given, else bfloat16 when ``OPTIONS.bf16`` and float32 otherwise."""
  import torch
  if dtype is not None:
    return dtype
  return torch.bfloat16 if OPTIONS.bf16 else torch.float32


def default_precision(precision=None, dtype=None):
  """`precision` if given, else ``OPTIONS.precision`` for float32 and "native" for bfloat16."""
  import torch
  if precision is not None:
    return precision
  return "native" if dtype == torch.bfloat16 else OPTIONS.precision


def default_reorder(reorder=None):
  """`reorder` if given, else ``OPTIONS.reorder``."""
  return OPTIONS.reorder if reorder is None else bool(reorder)


def missing_model_dependencies():
  """Modules the in-model patch needs that are not importable here."""
  return [m for m in ("jax", "haiku", "weathernext") if importlib.util.find_spec(m) is None]


def install():
  """Activates the HIP attention path (idempotent)."""
  global _enabled
  _enabled = True


def uninstall():
  """Restores the defaults."""
  global _enabled
  _enabled = False


def is_enabled():
  return _enabled
