"""Hilbert ordering and CSR live-tile list (oracle; test infrastructure only).

Restates ``pallas_attn.py:41-109`` of the reference in plain numpy:

* ``hilbert3``        Skilling's transpose algorithm ("Programming the Hilbert curve", AIP Conf.
                      Proc. 707, 2004) in 3-D, interleaved most-significant bit first with x[0]
                      leading each triple (``pallas_attn.py:41-68``).
* ``hilbert_order``   lat/lon -> unit xyz -> 10-bit quantised ints -> Hilbert index -> stable
                      argsort, non-finite points last (``pallas_attn.py:71-82``).
* ``build_tile_mask`` CSR over query blocks of the key tiles that hold at least one valid key,
                      tiles sorted by (query block, key block), one bitmask row per query row
                      (``pallas_attn.py:85-109``). The reference hard-wires 64x32 tiles with one
                      uint32 word per row; here the tile is block_q x block_k with block_k / 32
                      words per row (word w, bit j holds key kb*block_k + 32*w + j).
"""

import numpy as np
from scipy import sparse


def hilbert3(ints, bits):
  """3-D Hilbert index of non-negative int64[n, 3] coordinates < 2**bits."""
  x = [ints[:, i].astype(np.int64).copy() for i in range(3)]
  top = 1 << (bits - 1)
  # Inverse undo of excess work (Skilling): walk the bit planes from the top.
  q = top
  while q > 1:
    low = q - 1
    for i in range(3):
      set_ = (x[i] & q) != 0
      x[0] = np.where(set_, x[0] ^ low, x[0])
      swap = np.where(set_, 0, (x[0] ^ x[i]) & low)
      x[0] ^= swap
      x[i] ^= swap
    q >>= 1
  # Gray encode.
  x[1] ^= x[0]
  x[2] ^= x[1]
  flip = np.zeros_like(x[0])
  q = top
  while q > 1:
    flip = np.where((x[2] & q) != 0, flip ^ (q - 1), flip)
    q >>= 1
  for i in range(3):
    x[i] ^= flip
  code = np.zeros(len(x[0]), np.int64)
  for b in range(bits - 1, -1, -1):
    for i in range(3):
      code = (code << 1) | ((x[i] >> b) & 1)
  return code


def quantise_sphere(lat_deg, lon_deg, bits=10):
  """(ints int64[n, 3], finite bool[n]): unit xyz of each point (x towards lat 0 / lon 0, y towards
  lon 90, z towards the north pole) mapped from [-1, 1] to [0, 2**bits - 1], rounded half to even
  (``pallas_attn.py:75-78``)."""
  lat = np.deg2rad(np.asarray(lat_deg, np.float64).ravel())
  lon = np.deg2rad(np.asarray(lon_deg, np.float64).ravel())
  xyz = np.stack([np.cos(lat) * np.cos(lon), np.cos(lat) * np.sin(lon), np.sin(lat)], -1)
  finite = np.isfinite(xyz).all(-1)
  top = 2 ** bits - 1
  ints = np.clip(np.round((np.nan_to_num(xyz) + 1.0) / 2.0 * top), 0, top).astype(np.int64)
  return ints, finite


def hilbert_order(lat_deg, lon_deg, bits=10):
  """Permutation sorting points on the sphere along a 3-D Hilbert curve, non-finite points last."""
  ints, finite = quantise_sphere(lat_deg, lon_deg, bits)
  code = np.where(finite, hilbert3(ints, bits), np.iinfo(np.int64).max)
  return np.argsort(code, kind="stable")


def build_tile_mask(mask, block_q=128, block_k=128):
  """CSR tile list of a boolean [n_q, n_k] mask.

  Returns (tile_ptr int32[n_qb + 1], tile_kb int32[T], tile_bits uint32[T, block_q, block_k // 32]).
  """
  assert block_k % 32 == 0
  words = block_k // 32
  coo = sparse.coo_matrix(mask.astype(bool))
  rows, cols = coo.row.astype(np.int64), coo.col.astype(np.int64)
  n_q, n_k = mask.shape
  n_qb = -(-n_q // block_q)
  n_kb = -(-n_k // block_k)
  key = (rows // block_q) * n_kb + cols // block_k
  uniq, tile_of = np.unique(key, return_inverse=True)
  tile_qb, tile_kb = uniq // n_kb, uniq % n_kb
  within = cols % block_k
  bits = np.zeros((len(uniq), block_q, words), np.uint32)
  np.bitwise_or.at(bits, (tile_of, rows % block_q, within // 32),
                   np.left_shift(np.uint32(1), (within % 32).astype(np.uint32)))
  tile_ptr = np.zeros(n_qb + 1, np.int64)
  np.add.at(tile_ptr, tile_qb + 1, 1)
  return np.cumsum(tile_ptr).astype(np.int32), tile_kb.astype(np.int32), bits


def tiles_to_dense(tile_ptr, tile_kb, tile_bits, n_q, n_k, block_q=128, block_k=128):
  """Expand a tile list back to a dense boolean [n_q, n_k] mask."""
  n_qb = len(tile_ptr) - 1
  n_kb = int(tile_kb.max()) + 1 if len(tile_kb) else 1
  dense = np.zeros((n_qb * block_q, max(n_kb * block_k, n_k)), bool)
  shifts = np.arange(32, dtype=np.uint32)
  for qb in range(n_qb):
    for t in range(tile_ptr[qb], tile_ptr[qb + 1]):
      row_bits = ((tile_bits[t][:, :, None] >> shifts) & 1).astype(bool).reshape(block_q, -1)
      dense[qb * block_q:(qb + 1) * block_q, tile_kb[t] * block_k:(tile_kb[t] + 1) * block_k] = row_bits
  return dense[:n_q, :n_k]
