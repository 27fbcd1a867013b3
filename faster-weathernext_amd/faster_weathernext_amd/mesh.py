"""Icosahedral mesh, k-hop neighbourhood masks, Hilbert ordering and live-tile lists.

The reference takes WN2's mesh from weathernext (``TriangularMeshData.with_icosahedral_mesh``,
``scripts/attn_bench.py:26-33``) and builds the attention mask at trace time as
``adj_mat ** attention_k_hop`` (``patch.py:209``), the Hilbert permutation (``pallas_attn.py:71-82``)
and the tile list (``pallas_attn.py:85-109``) in numpy/scipy. Here:

* ``icosahedral_mesh(r)`` refines a regular icosahedron r times (4-way split at projected edge
  midpoints, new vertices numbered in order of first creation), vectorised in numpy.
* ``khop_mask``, ``hilbert_order`` and ``build_tile_mask`` run in the native library
  (multi-threaded breadth-first search, Skilling's Hilbert transform, per-block tile merge).
"""
import numpy as np
from scipy import sparse

from . import _native as nat

PHI = (1.0 + 5.0 ** 0.5) / 2.0


def icosahedron():
  """Unit icosahedron (vertices float64[12, 3], faces int64[20, 3], outward winding), with a face
  centre at each pole."""
  verts = []
  for c1 in (1.0, -1.0):
    for c2 in (PHI, -PHI):
      verts += [(c1, c2, 0.0), (0.0, c1, c2), (c2, 0.0, c1)]
  v = np.asarray(verts, np.float64) / np.hypot(1.0, PHI)
  angle = (np.pi - 2.0 * np.arcsin(PHI / np.sqrt(3.0))) / 2.0
  c, s = np.cos(angle), np.sin(angle)
  v = v @ np.array([[c, 0.0, s], [0.0, 1.0, 0.0], [-s, 0.0, c]])
  dist = np.linalg.norm(v[:, None] - v[None], axis=-1)
  edge = np.abs(dist - dist[dist > 1e-9].min()) < 1e-6
  tri = [(a, b, cc) for a in range(12) for b in range(a + 1, 12) for cc in range(b + 1, 12)
         if edge[a, b] and edge[b, cc] and edge[a, cc]]
  f = np.asarray(tri, np.int64)
  normal = np.cross(v[f[:, 1]] - v[f[:, 0]], v[f[:, 2]] - v[f[:, 0]])
  flip = np.einsum("fc,fc->f", normal, v[f].sum(1)) < 0
  f[flip] = f[flip][:, [0, 2, 1]]
  return v, f


def refine(vertices, faces):
  """One 4-way split of every face; midpoints numbered in order of first creation."""
  n = len(vertices)
  a, b, c = faces[:, 0], faces[:, 1], faces[:, 2]
  pairs = np.stack([np.stack([a, b], -1), np.stack([b, c], -1), np.stack([c, a], -1)], 1).reshape(-1, 2)
  key = pairs.min(1) * n + pairs.max(1)
  uniq, first, inverse = np.unique(key, return_index=True, return_inverse=True)
  rank = np.empty(len(uniq), np.int64)
  rank[np.argsort(first, kind="stable")] = np.arange(len(uniq))
  mid_id = (n + rank[inverse]).reshape(-1, 3)
  creation = np.argsort(first, kind="stable")
  ends = np.stack([uniq[creation] // n, uniq[creation] % n], -1)
  p = (vertices[ends[:, 0]] + vertices[ends[:, 1]]) / 2.0
  p /= np.sqrt((p * p).sum(1, keepdims=True))
  ab, bc, ca = mid_id[:, 0], mid_id[:, 1], mid_id[:, 2]
  out = np.stack([np.stack([a, ab, ca], -1), np.stack([ab, b, bc], -1), np.stack([ca, bc, c], -1),
                  np.stack([ab, bc, ca], -1)], 1).reshape(-1, 3)
  return np.concatenate([vertices, p]), out


def icosahedral_mesh(refinement):
  """(vertices float64[V, 3], faces int64[F, 3], lat_deg float64[V], lon_deg float64[V]);
  V = 10 * 4**r + 2 (642 at r = 3, 40,962 at r = 6)."""
  v, f = icosahedron()
  for _ in range(refinement):
    v, f = refine(v, f)
  lat = np.rad2deg(np.arcsin(np.clip(v[:, 2], -1.0, 1.0)))
  lon = np.rad2deg(np.arctan2(v[:, 1], v[:, 0]))
  return v, f, lat, lon


def adjacency(faces, n):
  """Boolean CSR adjacency of the mesh edges (both directions, no self edges), sorted indices."""
  s = faces[:, [0, 1, 2]].ravel()
  r = faces[:, [1, 2, 0]].ravel()
  a = sparse.csr_matrix((np.ones(2 * len(s), np.int8), (np.concatenate([s, r]), np.concatenate([r, s]))),
                        shape=(n, n))
  a = (a > 0).astype(bool).tocsr()
  a.sort_indices()
  return a


def khop_mask(adj, k):
  """Boolean CSR of the nodes within k hops of each node, itself included: the set of the
  reference's ``(adj + I) ** k`` (``patch.py:209``). Row i holds the nodes reachable from i in at
  most k steps along edges i -> j (adj[i, j] set), so a directed adjacency gives that power too."""
  adj = sparse.csr_matrix(adj)
  n = adj.shape[0]
  indptr = nat.as_c(adj.indptr, np.int64)
  indices = nat.as_c(adj.indices, np.int32)
  row_ptr = np.zeros(n + 1, np.int64)
  L = nat.lib()
  nat.check(L.fwn_khop_count(n, nat.ptr(indptr), nat.ptr(indices), int(k), nat.ptr(row_ptr)))
  idx = np.empty(int(row_ptr[-1]), np.int32)
  nat.check(L.fwn_khop_fill(n, nat.ptr(indptr), nat.ptr(indices), int(k), nat.ptr(row_ptr), nat.ptr(idx)))
  return sparse.csr_matrix((np.ones(len(idx), bool), idx, row_ptr), shape=(n, n))


def hilbert_order(lat_deg, lon_deg, bits=10):
  """Permutation sorting points on the sphere along a 3-D Hilbert curve, non-finite points last
  (``pallas_attn.hilbert_order``, ``pallas_attn.py:71-82``)."""
  lat = nat.as_c(np.asarray(lat_deg, np.float64).ravel(), np.float64)
  lon = nat.as_c(np.asarray(lon_deg, np.float64).ravel(), np.float64)
  if lat.shape != lon.shape:
    raise ValueError("lat and lon must have the same size")
  perm = np.empty(len(lat), np.int64)
  nat.check(nat.lib().fwn_hilbert_order(len(lat), nat.ptr(lat), nat.ptr(lon), int(bits), nat.ptr(perm)))
  return perm


def build_tile_mask(mask, block_q=nat.BLOCK, block_k=nat.BLOCK, *, perm=None):
  """CSR live-tile list of a boolean [n_rows, n_cols] mask at 128 x 128 tiles.

  The reference's signature (``pallas_attn.py:85``); its 64 x 32 tiles are not built here, so
  ``block_q`` and ``block_k`` must be 128 (ValueError otherwise).

  Returns (tile_ptr int32[n_blocks + 1], tile_kb int32[T], tile_bits uint32[T, 128, 4]): block i owns
  tiles tile_ptr[i]:tile_ptr[i+1]; tile t covers columns tile_kb[t]*128 + [0, 128) and bit j of word
  w of tile_bits[t, r] says whether row r of the block may attend to column tile_kb[t]*128 + 32w + j.
  With ``perm`` the list describes mask[perm][:, perm]. Same layout as the reference's
  ``build_tile_mask`` (``pallas_attn.py:85-109``) with 128-wide tiles (4 words per row).
  """
  if block_q != nat.BLOCK or block_k != nat.BLOCK:
    raise ValueError(f"tiles of {block_q} x {block_k}: the kernels use {nat.BLOCK} x {nat.BLOCK}")
  m = sparse.csr_matrix(mask)
  n_rows, n_cols = m.shape
  indptr = nat.as_c(m.indptr, np.int64)
  indices = nat.as_c(m.indices, np.int32)
  pp = None if perm is None else nat.as_c(perm, np.int64)
  n_blocks = -(-n_rows // nat.BLOCK)
  tile_ptr = np.zeros(n_blocks + 1, np.int32)
  L = nat.lib()
  nat.check(L.fwn_tiles_count(n_rows, n_cols, nat.ptr(indptr), nat.ptr(indices), nat.ptr(pp), nat.ptr(tile_ptr)))
  n_tiles = int(tile_ptr[-1])
  tile_kb = np.empty(n_tiles, np.int32)
  tile_bits = np.empty((n_tiles, nat.BLOCK, nat.BLOCK // 32), np.uint32)
  nat.check(L.fwn_tiles_fill(n_rows, n_cols, nat.ptr(indptr), nat.ptr(indices), nat.ptr(pp), nat.ptr(tile_ptr),
                             nat.ptr(tile_kb), nat.ptr(tile_bits)))
  return tile_ptr, tile_kb, tile_bits


def mesh_mask(refinement, k_hop, reorder=False):
  """The attention mask of one mesh transformer: (mask CSR, lat, lon, perm or None).

  The mask is the k-hop neighbourhood of the refined icosahedral mesh in subdivision order; with
  ``reorder`` the Hilbert permutation is returned as well (apply it with
  ``build_tile_mask(mask, perm=perm)``), as the reference's patched transformer does
  (``patch.py:208-214``).
  """
  v, f, lat, lon = icosahedral_mesh(refinement)
  mask = khop_mask(adjacency(f, len(v)), k_hop)
  perm = hilbert_order(lat, lon) if reorder else None
  return mask, lat, lon, perm
