"""Execution options and the attention dispatch of the drop-in switch.

Mirrors the attention slice of the reference's ``patch.py`` (``Options`` 50-79, ``attention_impl``
86-99, ``install``/``uninstall`` 727-758). Only the options that concern the attention path are
kept; the GNN / encoder / decoder blocking options of the reference are out of scope (they exist
to fit 8-32 GB cards).

The reference's patch swaps subclasses into the official ``weathernext`` modules so its
transformer calls ``pallas_attn.tiled_flash_attention``. Wiring this library into that JAX model
needs jax, haiku and weathernext plus an XLA FFI handler around the C ABI; ``install`` reports
which of them are missing instead of pretending to succeed.
"""
import dataclasses
import importlib.util


@dataclasses.dataclass
class Options:
  """Execution options (read when the model is traced)."""
  # Attention kernel: "hip" (the gfx950 kernels of this package) or "auto" (= "hip").
  attention: str = "auto"
  # Route every attention_type of the official configs to this implementation.
  replace_attention: bool = True
  # Process mesh nodes in Hilbert-curve order (exact; fewer live tiles).
  reorder: bool = True
  # Compute in bfloat16 with float32 accumulation instead of float32 MFMA.
  bf16: bool = False


OPTIONS = Options()
_enabled = False


def attention_impl():
  """The attention implementation ``enable()`` uses: always the HIP kernels."""
  if OPTIONS.attention not in ("auto", "hip"):
    raise ValueError(f"unknown attention implementation {OPTIONS.attention!r} (auto, hip)")
  return "hip"


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
