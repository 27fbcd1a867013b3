"""ctypes binding of libfwn_attn.so (the C ABI declared in include/fwn_attn.h and include/fwn_rows.h).

The library is loaded on first use from ``_lib/libfwn_attn.so`` next to this file. There is no
fallback: if it is missing or does not export every declared symbol, ``lib()`` raises.
"""
import ctypes
import os
import threading

import numpy as np

# FWN_LIB overrides the location (e.g. to compare two builds of the library).
LIB_PATH = os.environ.get("FWN_LIB") or os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "libfwn_attn.so")

BLOCK = 128
WAVES = 4
LANE_WORDS = WAVES * 64

F32 = 0
BF16 = 1

OK = 0
ERR_INVALID_ARG = 1
ERR_UNSUPPORTED = 2
ERR_TILES = 3
ERR_HIP = 4


class FwnError(RuntimeError):
  """A nonzero status from the C ABI; ``code`` is the fwn_status value."""

  def __init__(self, code, message):
    super().__init__(f"fwn status {code}: {message}")
    self.code = code


class AttnDesc(ctypes.Structure):
  _fields_ = [("batch", ctypes.c_int32), ("n", ctypes.c_int32), ("heads", ctypes.c_int32),
              ("head_dim", ctypes.c_int32), ("dtype", ctypes.c_int32), ("scale", ctypes.c_float),
              ("stride_b", ctypes.c_int64), ("stride_n", ctypes.c_int64), ("stride_h", ctypes.c_int64),
              ("ostride_b", ctypes.c_int64), ("ostride_n", ctypes.c_int64), ("ostride_h", ctypes.c_int64),
              ("precision", ctypes.c_int32), ("reserved", ctypes.c_int32)]


PREC_NATIVE = 0  # FWN_PREC_NATIVE: products in the tensors' dtype
PREC_BF16X3 = 1  # FWN_PREC_BF16X3: float32 tensors, products from three bf16 parts (forward and dS-exchange backward)


class Tiles(ctypes.Structure):
  _fields_ = [("n_blocks", ctypes.c_int32), ("n_tiles", ctypes.c_int32), ("ptr", ctypes.c_void_p),
              ("col", ctypes.c_void_p), ("lanes", ctypes.c_void_p), ("groups", ctypes.c_void_p),
              ("n_items", ctypes.c_int32), ("n_parts", ctypes.c_int32), ("n_split", ctypes.c_int32),
              ("n_work", ctypes.c_int32), ("items", ctypes.c_void_p), ("split", ctypes.c_void_p),
              ("halves", ctypes.c_void_p), ("work", ctypes.c_void_p), ("work_pairs", ctypes.c_int32),
              ("reserved", ctypes.c_int32)]


class DsMap(ctypes.Structure):
  _fields_ = [("n_units", ctypes.c_int64), ("ubase", ctypes.c_void_p), ("tmap", ctypes.c_void_p),
              ("unit_keys", ctypes.c_int32), ("reserved", ctypes.c_int32)]


ITEM_TILES = 64  # FWN_ITEM_TILES: default longest run of tiles per work item
ORDER_ITEMS, ORDER_BALANCED, ORDER_MAKESPAN = 0, 1, 2  # FWN_ORDER_*
SCRATCH_BYTES = 64 << 20  # FWN_SCRATCH_BYTES: static scratch of fwn_attn_fwd_launch_noalloc


class RowsDesc(ctypes.Structure):
  _fields_ = [("batch", ctypes.c_int32), ("n", ctypes.c_int32), ("channels", ctypes.c_int32),
              ("dtype", ctypes.c_int32), ("eps", ctypes.c_float)]


ROWS_MAX_CHANNELS = 4096  # FWN_ROWS_MAX_CHANNELS


_P = ctypes.c_void_p
_I32, _I64, _U64, _F = ctypes.c_int32, ctypes.c_int64, ctypes.c_uint64, ctypes.c_float
_DESC = ctypes.POINTER(AttnDesc)
_TILES = ctypes.POINTER(Tiles)
_ROWS = ctypes.POINTER(RowsDesc)
_DS = ctypes.POINTER(DsMap)

# name -> argtypes, every entry point of include/fwn_attn.h and include/fwn_rows.h
SIGNATURES = {
    "fwn_last_error": [],
    "fwn_khop_count": [_I32, _P, _P, _I32, _P],
    "fwn_khop_fill": [_I32, _P, _P, _I32, _P, _P],
    "fwn_hilbert_order": [_I64, _P, _P, _I32, _P],
    "fwn_tiles_count": [_I32, _I32, _P, _P, _P, _P],
    "fwn_tiles_fill": [_I32, _I32, _P, _P, _P, _P, _P, _P],
    "fwn_tiles_prepare": [_I32, _I32, _I32, _P, _P, _P, _P, _P, _P],
    "fwn_tiles_schedule_count": [_I32, _P, _I32, _P, _P, _P],
    "fwn_tiles_schedule_fill": [_I32, _P, _I32, _P, _P],
    "fwn_tiles_order_count": [_I32, _P, _P, _I32, _I32, _I32, _I32, _I32, _P],
    "fwn_tiles_order_fill": [_I32, _P, _P, _I32, _I32, _I32, _I32, _I32, _P],
    "fwn_attn_workspace_size": [_DESC, _TILES, _P],
    "fwn_attn_fwd_launch": [_DESC, _P, _P, _P, _TILES, _P, _P, _P, _U64, _P],
    "fwn_attn_fwd_launch_noalloc": [_DESC, _P, _P, _P, _TILES, _P, _P, _P],
    "fwn_attn_bwd_delta_launch": [_DESC, _P, _P, _P, _P],
    "fwn_attn_bwd_dq_launch": [_DESC, _P, _P, _P, _P, _P, _P, _TILES, _P, _P, _U64, _P],
    "fwn_attn_bwd_dkv_launch": [_DESC, _P, _P, _P, _P, _P, _P, _TILES, _P, _P, _P, _U64, _P],
    "fwn_attn_bwd_launch": [_DESC, _P, _P, _P, _P, _P, _P, _P, _TILES, _TILES, _P, _P, _P, _P, _U64, _P],
    "fwn_tiles_ds_map": [_I32, _P, _P, _P, _P, _P, _P, _I32, _P, _P, _P],
    "fwn_attn_ds_bytes": [_DESC, _DS, _P],
    "fwn_attn_bwd_dkv_ds_launch": [_DESC, _P, _P, _P, _P, _P, _P, _TILES, _DS, _P, _P, _P, _U64, _P, _U64, _P],
    "fwn_attn_bwd_dq_ds_launch": [_DESC, _P, _P, _U64, _TILES, _DS, _P, _P, _U64, _P],
    "fwn_attn_bwd_ds_launch": [_DESC, _P, _P, _P, _P, _P, _P, _P, _TILES, _TILES, _DS, _P, _P, _P, _P, _U64, _P, _U64,
                               _P],
    "fwn_rows_gather_norm_launch": [_ROWS, _P, _P, _P, _P, _P],
    "fwn_rows_norm_scatter_launch": [_ROWS, _P, _P, _P, _P, _P, _P],
    "fwn_rows_norm_affine_launch": [_ROWS, _P, _P, _P, _P, _P],
    "fwn_rows_add_norm_affine_launch": [_ROWS, _P, _P, _P, _P, _P, _P, _P],
}

_lock = threading.Lock()
_lib = None


def lib():
  """The loaded library (raises if it was not built)."""
  global _lib
  with _lock:
    if _lib is None:
      if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} not found: build it with `python faster-weathernext_amd/build.py`")
      handle = ctypes.CDLL(LIB_PATH)
      for name, args in SIGNATURES.items():
        fn = getattr(handle, name)  # AttributeError names a missing export
        fn.argtypes = args
        fn.restype = ctypes.c_char_p if name == "fwn_last_error" else ctypes.c_int
      _lib = handle
  return _lib


def check(status):
  """Raises FwnError for a nonzero status, with the library's thread-local message."""
  if status != OK:
    raise FwnError(status, lib().fwn_last_error().decode(errors="replace"))


def ptr(a):
  """Address of a numpy array's data (None for empty arrays)."""
  if a is None:
    return None
  return a.ctypes.data if a.size else None


def as_c(a, dtype):
  return np.ascontiguousarray(a, dtype=dtype)
