"""Execution options and the attention dispatch of the drop-in switch.

Mirrors the attention slice of the reference's ``patch.py`` (``Options`` 50-79, ``attention_impl``
86-99, ``install``/``uninstall`` 727-758). ``Options`` carries every field of the reference's, with
its default, so ``enable(**options)`` written for the reference is accepted; the fields that
concern other parts of the reference (the XLA chunked attention, the GNN / encoder / decoder
blocking, the Haiku layer loop, rematerialisation) have no effect here and say so below.

The options are read when a model is built: ``MeshTransformer`` takes its node order from
``reorder`` and, with ``TiledMHA``, its parameter and activation dtype from ``bf16`` and its
product precision from ``precision`` / ``strict_fp32`` when the caller passes none.

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
  """Execution options (read when a model is built). The first nine fields are the reference's
  (``patch.py:50-79``), with its defaults; the last two are this build's."""
  # Attention kernel: "hip" (the gfx950 kernels of this package) or "auto" (= "hip" on gfx950).
  attention: str = "auto"
  # Reference: route every attention type of the official configs to the fast kernel. This
  # library has one attention implementation, so there is nothing to route; no effect.
  replace_attention: bool = True
  # Process mesh nodes in Hilbert-curve order (exact; fewer live tiles). MeshTransformer's default.
  reorder: bool = True
  # IEEE float32 products for float32 tensors, whatever the float32 matmul precision (the
  # reference's switch away from its tensor-core dots). See resolve_precision.
  strict_fp32: bool = False
  # Reference: queries per chunk of its XLA chunked attention. There is no XLA path here (the
  # chunked path exists only as the test oracle); no effect.
  attn_chunk: int = 512
  # Reference: grid points / edges per block of its memory-blocked GNN, encoder and decoder,
  # which this library does not contain (they exist to fit 8-32 GB cards); no effect.
  grid_chunk: int = 32768
  edge_chunk: int = 65536
  # Reference: run the 24 layers as hk.scan + hk.switch. MeshTransformer runs its layers in a
  # Python loop over one shared tile list either way; no effect.
  layer_loop: bool = True
  # Reference: rematerialise blocks / layers / chunks in the backward, and run the stacked batch
  # one member at a time. The attention backward here already recomputes P from the saved
  # log-sum-exp and keeps no per-chunk intermediates; no effect.
  remat: bool = False
  sequential_samples: bool = False
  # bfloat16 parameters and activations with float32 accumulation instead of float32 (fp32 MFMA).
  # MeshTransformer's and TiledMHA's default dtype.
  bf16: bool = False
  # Products of the attention kernels on float32 tensors: None (from strict_fp32 and torch's
  # float32 matmul precision, see resolve_precision), "native" (IEEE float32 products) or
  # "bf16x3" (three bf16 products per float32 product, about 16 significant bits per operand).
  # bfloat16 tensors always take bf16 products.
  precision: str = None


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


PRECISIONS = ("native", "bf16x3")


def resolve_precision(precision=None, dtype=None, strict_fp32=None):
  """The product precision ("native" or "bf16x3") of an attention call on `dtype` tensors.

  The reference picks its dot algorithm from JAX's default matmul precision and strict_fp32
  (``pallas_attn.py:336-341``): under "highest" IEEE float32 dots if strict_fp32, else 3xTF32;
  otherwise one TF32 dot. Here the same choice reads torch's float32 matmul precision
  (``torch.get_float32_matmul_precision``): under "highest" (torch's default, documented as full
  float32 products) the IEEE float32 kernels; under "high" or "medium" (documented as TF32 or
  "the sum of two bfloat16 numbers") the bf16x3 kernels, which are gfx950's matrix-core float32
  path (it has no TF32 MFMA), unless strict_fp32 asks for IEEE products. An explicit `precision`
  wins, but strict_fp32 with "bf16x3" is refused. bfloat16 tensors always take bf16 products
  ("native"; an explicit "bf16x3" is refused, the option is not applied to them). strict_fp32 None takes ``OPTIONS.strict_fp32``; `precision` None takes
  ``OPTIONS.precision`` when that is set."""
  import torch
  strict = OPTIONS.strict_fp32 if strict_fp32 is None else bool(strict_fp32)
  if precision is not None and precision not in PRECISIONS:
    raise ValueError(f"precision {precision!r}: one of {PRECISIONS}")
  if dtype == torch.bfloat16:
    if precision == "bf16x3":
      raise TypeError("precision 'bf16x3' needs float32 tensors")
    return "native"
  if precision is None:
    precision = OPTIONS.precision
  if strict:
    if precision not in (None, "native"):
      raise ValueError("strict_fp32 asks for IEEE float32 products: precision must be 'native'")
    return "native"
  if precision is not None:
    return precision
  return "native" if torch.get_float32_matmul_precision() == "highest" else "bf16x3"


def default_precision(precision=None, dtype=None):
  """`precision` if given, else the resolved precision for `dtype` (see resolve_precision)."""
  return resolve_precision(precision, dtype)


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
