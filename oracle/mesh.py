"""Icosahedral mesh and k-hop neighbourhood mask (oracle; test infrastructure only).

The reference builds WN2's mesh with weathernext's
``TriangularMeshData.with_icosahedral_mesh(splits_list=[2] * 6)`` and the attention mask as
``(adj + I) ** k_hop`` over the face edges (``scripts/attn_bench.py:26-33``; in the model
``adj_mat ** attention_k_hop`` on the mesh adjacency with self edges, ``patch.py:209``). weathernext
is not vendored, so the mesh here is an independent construction of the same object: a regular
icosahedron refined r times by splitting every triangle into four at its edge midpoints
(projected to the unit sphere). New vertices are numbered in order of first creation while the
faces are visited in order, which gives the "vertex order from the deterministic subdivision".
The neighbourhood *sizes* depend only on the graph, which is the same for any such refinement;
the vertex numbering and orientation of the official mesh are not pinned here.
"""

import numpy as np
from scipy import sparse

PHI = (1.0 + 5.0 ** 0.5) / 2.0


def icosahedron():
  """Unit icosahedron: (vertices float64[12, 3], faces int64[20, 3]) with outward winding.

  Vertices are the cyclic permutations of (0, +-1, +-phi), rotated about the y axis by
  (pi - dihedral) / 2, which puts a face centre at each pole (the orientation GraphCast-style
  meshes use). Faces are found from the geometry (triples of mutually adjacent vertices).
  """
  verts = []
  for c1 in (1.0, -1.0):
    for c2 in (PHI, -PHI):
      verts += [(c1, c2, 0.0), (0.0, c1, c2), (c2, 0.0, c1)]
  v = np.asarray(verts, np.float64) / np.hypot(1.0, PHI)
  dihedral = 2.0 * np.arcsin(PHI / np.sqrt(3.0))
  a = (np.pi - dihedral) / 2.0
  rot = np.array([[np.cos(a), 0.0, np.sin(a)], [0.0, 1.0, 0.0], [-np.sin(a), 0.0, np.cos(a)]])
  v = v @ rot
  d = np.linalg.norm(v[:, None] - v[None], axis=-1)
  edge = d[d > 1e-9].min()
  adj = np.abs(d - edge) < 1e-6
  faces = []
  for i in range(12):
    for j in range(i + 1, 12):
      for k in range(j + 1, 12):
        if adj[i, j] and adj[j, k] and adj[i, k]:
          f = (i, j, k)
          if np.dot(np.cross(v[j] - v[i], v[k] - v[i]), v[i] + v[j] + v[k]) < 0:
            f = (i, k, j)
          faces.append(f)
  return v, np.asarray(faces, np.int64)


def refine(vertices, faces):
  """One 4-way split of every triangle; midpoints are appended in order of first creation."""
  verts = [tuple(p) for p in vertices]
  mid = {}

  def child(a, b):
    key = (a, b) if a < b else (b, a)
    if key not in mid:
      p = (np.asarray(verts[a]) + np.asarray(verts[b])) / 2.0
      verts.append(tuple(p / np.linalg.norm(p)))
      mid[key] = len(verts) - 1
    return mid[key]

  out = []
  for a, b, c in faces:
    ab, bc, ca = child(a, b), child(b, c), child(c, a)
    out += [(a, ab, ca), (ab, b, bc), (ca, bc, c), (ab, bc, ca)]
  return np.asarray(verts, np.float64), np.asarray(out, np.int64)


def icosahedral_mesh(refinement):
  """(vertices float64[V, 3], faces int64[F, 3], lat_deg float64[V], lon_deg float64[V])."""
  v, f = icosahedron()
  for _ in range(refinement):
    v, f = refine(v, f)
  lat = np.rad2deg(np.arcsin(np.clip(v[:, 2], -1.0, 1.0)))
  lon = np.rad2deg(np.arctan2(v[:, 1], v[:, 0]))
  return v, f, lat, lon


def adjacency(faces, n):
  """Boolean CSR adjacency of the face edges (both directions), without self edges."""
  s = np.concatenate([faces[:, 0], faces[:, 1], faces[:, 2]])
  r = np.concatenate([faces[:, 1], faces[:, 2], faces[:, 0]])
  a = sparse.csr_matrix((np.ones(2 * len(s), np.int8), (np.concatenate([s, r]), np.concatenate([r, s]))),
                        shape=(n, n))
  return (a > 0).astype(bool).tocsr()


def khop_mask(adj, k):
  """(adj + I)^k as a boolean CSR: keys within k hops of each query, the query included.

  Same set as the reference's ``(adj + I) ** k`` (``scripts/attn_bench.py:32``); computed by
  repeated squaring with re-binarisation so walk counts never overflow.
  """
  n = adj.shape[0]
  base = (adj.astype(bool) + sparse.identity(n, dtype=bool, format="csr")).astype(np.float32).tocsr()
  result = None
  power = base
  while k:
    if k & 1:
      result = power if result is None else ((result @ power) > 0).astype(np.float32).tocsr()
    k >>= 1
    if k:
      power = ((power @ power) > 0).astype(np.float32).tocsr()
  if result is None:
    result = sparse.identity(n, dtype=np.float32, format="csr")
  out = (result > 0).astype(bool).tocsr()
  out.sort_indices()
  return out
