"""On-disk cache of live-tile lists.

The reference rebuilds the k-hop mask and its tile list in every process, at trace time
(``patch.py:208-219``; 35 s for the 32-hop refinement-6 mask with scipy,
``docs/results/attn_bwd/attn_bwd_default_rtx5090.txt:3``). The native pipeline here takes well
under a second. This cache removes even that from repeated runs, and it lets a process without
the mesh code load the list.

File format (little endian), one tile list per file:

    offset  size  field
         0     8  magic b"FWNTILES"
         8     4  format version (1)
        12     4  n_rows (queries)
        16     4  n_cols (keys)
        20     4  k_hop (-1 when the mask did not come from a k-hop neighbourhood)
        24     4  order (0 = as given, 1 = Hilbert-permuted)
        28     4  block (128)
        32     8  key: 64-bit BLAKE2b digest of the mask (CSR arrays) and the permutation
        40     4  n_blocks
        44     4  n_tiles
        48        tile_ptr int32[n_blocks + 1], tile_col int32[n_tiles],
                  tile_bits uint32[n_tiles * 128 * 4]

A file whose header does not match what the caller expects (other key, shape, block, version or
a truncated body) is ignored and rebuilt.
"""
import hashlib
import os
import struct

import numpy as np

from . import _native as nat
from .mesh import build_tile_mask, khop_mask

MAGIC = b"FWNTILES"
VERSION = 1
_HEADER = struct.Struct("<8sIiiiiiQii")  # 48 bytes, offsets as documented above


def mask_key(mask, perm=None, k_hop=None):
  """64-bit digest of a boolean CSR matrix (a mask, or an adjacency together with `k_hop`) and an
  optional permutation."""
  from scipy import sparse
  m = sparse.csr_matrix(mask)
  m.sort_indices()
  h = hashlib.blake2b(digest_size=8)
  h.update(np.asarray(m.shape + ((-1 if k_hop is None else int(k_hop)),), np.int64).tobytes())
  h.update(np.ascontiguousarray(m.indptr, np.int64).tobytes())
  h.update(np.ascontiguousarray(m.indices, np.int32).tobytes())
  if perm is not None:
    h.update(np.ascontiguousarray(perm, np.int64).tobytes())
  return int.from_bytes(h.digest(), "little")


def save(path, tile_ptr, tile_kb, tile_bits, *, n_rows, n_cols, key, k_hop=-1, order=0):
  """Writes one tile list (atomically: a temporary file renamed over `path`)."""
  tile_ptr = np.ascontiguousarray(tile_ptr, np.int32)
  tile_kb = np.ascontiguousarray(tile_kb, np.int32)
  tile_bits = np.ascontiguousarray(tile_bits, np.uint32)
  n_blocks, n_tiles = len(tile_ptr) - 1, len(tile_kb)
  if tile_bits.size != n_tiles * nat.BLOCK * (nat.BLOCK // 32):
    raise ValueError("tile_bits does not hold 128 x 4 words per tile")
  head = _HEADER.pack(MAGIC, VERSION, int(n_rows), int(n_cols), int(k_hop), int(order), nat.BLOCK,
                      int(key) & (2 ** 64 - 1), n_blocks, n_tiles)
  tmp = f"{path}.tmp{os.getpid()}"
  with open(tmp, "wb") as f:
    f.write(head)
    f.write(tile_ptr.tobytes())
    f.write(tile_kb.tobytes())
    f.write(tile_bits.tobytes())
  os.replace(tmp, path)


def load(path, *, n_rows, n_cols, key):
  """(tile_ptr, tile_kb, tile_bits) from `path`, or None if it is missing or does not match."""
  try:
    with open(path, "rb") as f:
      raw = f.read()
  except OSError:
    return None
  if len(raw) < _HEADER.size:
    return None
  magic, version, nr, nc, _, _, block, fkey, n_blocks, n_tiles = _HEADER.unpack_from(raw)
  if (magic != MAGIC or version != VERSION or block != nat.BLOCK or nr != n_rows or nc != n_cols or
      fkey != (int(key) & (2 ** 64 - 1)) or n_blocks != -(-n_rows // nat.BLOCK) or n_tiles < 0):
    return None
  words = nat.BLOCK * (nat.BLOCK // 32)
  sizes = [(n_blocks + 1) * 4, n_tiles * 4, n_tiles * words * 4]
  if len(raw) != _HEADER.size + sum(sizes):
    return None
  off = _HEADER.size
  tile_ptr = np.frombuffer(raw, np.int32, n_blocks + 1, off).copy()
  off += sizes[0]
  tile_kb = np.frombuffer(raw, np.int32, n_tiles, off).copy()
  off += sizes[1]
  tile_bits = np.frombuffer(raw, np.uint32, n_tiles * words, off).copy().reshape(n_tiles, nat.BLOCK, -1)
  if tile_ptr[0] != 0 or tile_ptr[-1] != n_tiles or np.any(np.diff(tile_ptr) < 0):
    return None
  return tile_ptr, tile_kb, tile_bits


def cached_tile_mask(mask, perm=None, *, cache_dir, k_hop=-1):
  """build_tile_mask(mask, perm=perm) through a cache file in `cache_dir` keyed by the mask's content.

  Returns (tile_ptr, tile_kb, tile_bits, hit)."""
  n_rows, n_cols = mask.shape
  key = mask_key(mask, perm)
  os.makedirs(cache_dir, exist_ok=True)
  path = os.path.join(cache_dir, f"tiles_{n_rows}x{n_cols}_{key:016x}.fwnt")
  got = load(path, n_rows=n_rows, n_cols=n_cols, key=key)
  if got is not None:
    return (*got, True)
  tp, kb, bits = build_tile_mask(mask, perm=perm)
  save(path, tp, kb, bits, n_rows=n_rows, n_cols=n_cols, key=key, k_hop=k_hop, order=int(perm is not None))
  return tp, kb, bits, False


def cached_khop_tiles(adj, k_hop, perm=None, *, cache_dir):
  """The tile list of the k-hop mask of adjacency `adj` (permuted as mask[perm][:, perm]) through
  a cache file keyed by the adjacency, k and the permutation: a hit skips both the k-hop mask and
  the tile list. Returns (tile_ptr, tile_kb, tile_bits, hit)."""
  n = adj.shape[0]
  key = mask_key(adj, perm, k_hop)
  os.makedirs(cache_dir, exist_ok=True)
  path = os.path.join(cache_dir, f"khop{int(k_hop)}_{n}_{key:016x}.fwnt")
  got = load(path, n_rows=n, n_cols=n, key=key)
  if got is not None:
    return (*got, True)
  tp, kb, bits = build_tile_mask(khop_mask(adj, k_hop), perm=perm)
  save(path, tp, kb, bits, n_rows=n, n_cols=n, key=key, k_hop=k_hop, order=int(perm is not None))
  return tp, kb, bits, False
