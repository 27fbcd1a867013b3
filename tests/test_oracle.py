"""Pins the CPU oracle against closed forms, brute force and the reference's own invariants.

Each check is chosen so that a plausible slip in the oracle (a dropped term, a wrong sign or
index, a transposed operand) fails it; none of them retypes the oracle's formula.
"""
import itertools

import numpy as np
import pytest
from scipy import sparse

import hilbert_cases as HC
from oracle import attention as A
from oracle import mesh, rows, tiles


def _random_mask(n, density, seed, symmetric=False):
  m = sparse.random(n, n, density=density, random_state=seed, format="csr").astype(bool)
  if symmetric:
    m = m + m.T
  return (m + sparse.identity(n, dtype=bool, format="csr")).tocsr().astype(bool)


# ---------------------------------------------------------------------------------------------
# dense attention and gradients


def test_dense_attention_matches_row_by_row_softmax():
  rng = np.random.default_rng(11)
  b, n, h, d = 2, 17, 3, 5
  q, k, v = (rng.standard_normal((b, n, h, d)) for _ in range(3))
  mask = _random_mask(n, 0.3, 1).toarray()
  scale = 0.37
  out = A.dense_attention(q, k, v, mask, scale)
  lse = A.dense_lse(q, k, mask, scale)
  for bi, hi, i in itertools.product(range(b), range(h), range(n)):
    keys = np.flatnonzero(mask[i])
    logits = [scale * sum(q[bi, i, hi, c] * k[bi, j, hi, c] for c in range(d)) for j in keys]
    mx = max(logits)
    w = [np.exp(x - mx) for x in logits]
    tot = sum(w)
    for c in range(d):
      ref = sum(wj * v[bi, j, hi, c] for wj, j in zip(w, keys)) / tot
      assert abs(out[bi, i, hi, c] - ref) < 1e-12
    assert abs(lse[bi, hi, i] - (mx + np.log(tot))) < 1e-12


def test_dense_attention_invariants():
  rng = np.random.default_rng(12)
  b, n, h, d = 1, 40, 2, 8
  q, k, v = (rng.standard_normal((b, n, h, d)) for _ in range(3))
  mask = _random_mask(n, 0.2, 2).toarray()
  # Constant values -> constant output (rows of P sum to 1).
  ones = np.ones_like(v)
  np.testing.assert_allclose(A.dense_attention(q, k, ones, mask, 0.5), ones, atol=1e-13)
  # Masked keys have no influence on the output.
  k2, v2 = k.copy(), v.copy()
  k2[:, ~mask[0]] += 100.0
  v2[:, ~mask[0]] -= 7.0
  np.testing.assert_allclose(A.dense_attention(q, k2, v2, mask, 0.5)[:, 0],
                             A.dense_attention(q, k, v, mask, 0.5)[:, 0], atol=1e-12)


def test_dense_grads_match_finite_differences():
  rng = np.random.default_rng(13)
  b, n, h, d = 1, 9, 2, 3
  q, k, v, do = (rng.standard_normal((b, n, h, d)) for _ in range(4))
  mask = _random_mask(n, 0.35, 3).toarray()
  scale = 0.8
  grads = A.dense_grads(q, k, v, do, mask, scale)
  loss = lambda q_, k_, v_: float((A.dense_attention(q_, k_, v_, mask, scale) * do).sum())
  eps = 1e-6
  for which, g in enumerate(grads):
    for idx in [(0, 0, 0, 0), (0, 3, 1, 2), (0, 8, 1, 1), (0, 5, 0, 2)]:
      args = [q.copy(), k.copy(), v.copy()]
      args[which][idx] += eps
      up = loss(*args)
      args[which][idx] -= 2 * eps
      dn = loss(*args)
      assert abs((up - dn) / (2 * eps) - g[idx]) < 1e-7, (which, idx)


def test_dense_grads_masked_keys_get_nothing():
  rng = np.random.default_rng(14)
  n = 30
  q, k, v, do = (rng.standard_normal((1, n, 1, 4)) for _ in range(4))
  mask = np.eye(n, dtype=bool)
  mask[:10, :20] = True  # keys 20.. are visible only to themselves
  dq, dk, dv = A.dense_grads(q, k, v, do, mask, 1.0)
  # A key seen only by its own row with weight 1 has dV = dO of that row and dK = 0.
  np.testing.assert_allclose(dv[:, 20:], do[:, 20:], atol=1e-13)
  np.testing.assert_allclose(dk[:, 20:], 0.0, atol=1e-13)
  np.testing.assert_allclose(dq[:, 20:], 0.0, atol=1e-13)


# ---------------------------------------------------------------------------------------------
# reference XLA chunked path


def test_chunked_mask_roundtrip():
  # tests/test_masks.py:55-66 of the reference: banded mask, chunk 64.
  n, chunk = 700, 64
  i, j = np.meshgrid(np.arange(n), np.arange(n), indexing="ij")
  m = sparse.csr_matrix(np.abs(i - j) <= 40)
  starts, bits, window, n_kv = A.build_chunked_mask(m, chunk)
  dense = np.zeros((len(starts) * chunk, n_kv), bool)
  unpacked = np.unpackbits(bits, axis=-1, count=window, bitorder="little").astype(bool)
  for c, s in enumerate(starts):
    dense[c * chunk:(c + 1) * chunk, s:s + window] = unpacked[c]
  np.testing.assert_array_equal(dense[:n, :n], m.toarray())
  assert window % 128 == 0


@pytest.mark.parametrize("dtype,tol", [(np.float64, 1e-12), (np.float32, 2e-6)])
def test_chunked_path_equals_dense(dtype, tol):
  rng = np.random.default_rng(15)
  b, n, h, d = 2, 300, 2, 16
  q, k, v, do = (rng.standard_normal((b, n, h, d)).astype(dtype) for _ in range(4))
  m = _random_mask(n, 0.05, 4, symmetric=True)
  starts, bits, window, n_kv = A.build_chunked_mask(m, 64)
  scale = d ** -0.5
  out = A.chunked_attention(q, k, v, starts, bits, window, n_kv, 64, scale)
  ref = A.dense_attention(q, k, v, m.toarray(), scale)
  assert A.rel_rms(out, ref) < tol
  got = A.chunked_attention_grads(q, k, v, do, starts, bits, window, n_kv, 64, scale)
  for g, r in zip(got, A.dense_grads(q, k, v, do, m.toarray(), scale)):
    assert A.rel_rms(g, r) < tol


# ---------------------------------------------------------------------------------------------
# mesh and k-hop mask


@pytest.mark.parametrize("r", [0, 1, 2, 3, 4])
def test_mesh_closed_forms(r):
  v, f, lat, lon = mesh.icosahedral_mesh(r)
  n = len(v)
  assert n == 10 * 4 ** r + 2 and len(f) == 20 * 4 ** r
  adj = mesh.adjacency(f, n)
  assert adj.nnz == 2 * 30 * 4 ** r                    # E = 30 * 4^r undirected edges
  assert n - adj.nnz // 2 + len(f) == 2                 # Euler characteristic of the sphere
  deg = np.diff(adj.indptr)
  assert (deg == 5).sum() == 12 and (deg == 6).sum() == n - 12
  np.testing.assert_allclose(np.linalg.norm(v, axis=1), 1.0, atol=1e-14)
  # Outward winding: every face normal points away from the centre.
  nrm = np.cross(v[f[:, 1]] - v[f[:, 0]], v[f[:, 2]] - v[f[:, 0]])
  assert (np.einsum("fc,fc->f", nrm, v[f].sum(1)) > 0).all()
  assert np.all(np.abs(lat) <= 90) and np.all(np.abs(lon) <= 180)


def _bfs_ball(adj, src, k):
  seen = {src}
  frontier = [src]
  for _ in range(k):
    nxt = []
    for u in frontier:
      for w in adj.indices[adj.indptr[u]:adj.indptr[u + 1]]:
        if w not in seen:
          seen.add(w)
          nxt.append(w)
    frontier = nxt
  return seen


@pytest.mark.parametrize("k", [0, 1, 2, 3, 5])
def test_khop_equals_brute_force_bfs(k):
  v, f, _, _ = mesh.icosahedral_mesh(2)
  adj = mesh.adjacency(f, len(v))
  m = mesh.khop_mask(adj, k)
  assert (m != m.T).nnz == 0
  for src in range(len(v)):
    assert set(m.indices[m.indptr[src]:m.indptr[src + 1]].tolist()) == _bfs_ball(adj, src, k)


def test_khop_hexagonal_closed_form_away_from_pentagons():
  v, f, _, _ = mesh.icosahedral_mesh(5)
  adj = mesh.adjacency(f, len(v))
  deg = np.diff(adj.indptr)
  pent = np.flatnonzero(deg == 5)
  # Graph distance of every node to the nearest pentagon.
  dist = np.full(len(v), -1)
  dist[pent] = 0
  frontier = list(pent)
  while frontier:
    nxt = []
    for u in frontier:
      for w in adj.indices[adj.indptr[u]:adj.indptr[u + 1]]:
        if dist[w] < 0:
          dist[w] = dist[u] + 1
          nxt.append(w)
    frontier = nxt
  for k in (1, 2, 4, 8):
    m = mesh.khop_mask(adj, k)
    sizes = np.diff(m.indptr)
    far = dist > k
    assert far.any()
    assert (sizes[far] == 1 + 3 * k * (k + 1)).all(), k
    assert (sizes[~far] <= 1 + 3 * k * (k + 1)).all()


# ---------------------------------------------------------------------------------------------
# Hilbert order and tile list


@pytest.mark.parametrize("bits", [1, 2, 3])
def test_hilbert3_is_a_hilbert_curve(bits):
  side = 1 << bits
  cells = np.array(list(itertools.product(range(side), repeat=3)), np.int64)
  code = tiles.hilbert3(cells, bits)
  assert sorted(code.tolist()) == list(range(side ** 3))      # bijection onto [0, 8^bits)
  path = cells[np.argsort(code)]
  assert (np.abs(np.diff(path, axis=0)).sum(1) == 1).all()     # unit steps along the curve
  assert (path[0] == 0).all()                                  # starts at the origin


@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_hilbert3_inverts_skillings_transpose_to_axes(bits):
  # The paper's other routine (index -> axes), written independently in hilbert_cases: every index
  # must come back, so hilbert3 is exactly Skilling's AxestoTranspose with axis 0 leading.
  h = np.arange(8 ** bits)
  cells = HC.skilling_transpose_to_axes(h, bits)
  np.testing.assert_array_equal(tiles.hilbert3(cells, bits), h)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_hilbert_order_octant_centres_follow_gray_code(seed):
  lat, lon, want = HC.octant_case(seed)
  np.testing.assert_array_equal(tiles.hilbert_order(lat, lon), want)


def _planted_order(lat, lon, axes=(0, 1, 2), signs=(1, 1, 1)):
  """The oracle's order with a planted slip: xyz axes permuted and / or negated."""
  lat, lon = np.asarray(lat, np.float64), np.asarray(lon, np.float64)
  ints, _ = tiles.quantise_sphere(lat, lon)
  ints = ints[:, list(axes)]
  for a, s in enumerate(signs):
    if s < 0:
      ints[:, a] = 1023 - ints[:, a]
  return np.argsort(tiles.hilbert3(ints, 10), kind="stable")


@pytest.mark.parametrize("axes,signs", [(p, (1, 1, 1)) for p in itertools.permutations(range(3)) if p != (0, 1, 2)] +
                         [((0, 1, 2), s) for s in ((-1, 1, 1), (1, -1, 1), (1, 1, -1))])
def test_octant_check_catches_planted_axis_slips(axes, signs):
  # Each of the five wrong axis orders, and each negated axis, fails the octant known answer.
  lat, lon, want = HC.octant_case(0)
  assert (_planted_order(lat, lon) == want).all()
  assert not (_planted_order(lat, lon, axes, signs) == want).all()


def test_hilbert_quantises_axis_points():
  names = list(HC.AXIS_POINTS)
  lat, lon = np.array([HC.AXIS_POINTS[k] for k in names]).T
  ints, finite = tiles.quantise_sphere(lat, lon, 10)
  assert finite.all()
  assert [tuple(c) for c in ints.tolist()] == [HC.AXIS_CELLS[k] for k in names]
  assert HC.axis_order_ok(tiles.hilbert_order(lat, lon), names)


def test_hilbert_order_is_permutation_and_local():
  # tests/test_masks.py:39-52 of the reference.
  rng = np.random.default_rng(0)
  lat, lon = rng.uniform(-90, 90, 5000), rng.uniform(0, 360, 5000)
  lat[:3] = np.nan
  perm = tiles.hilbert_order(lat, lon)
  assert sorted(perm.tolist()) == list(range(5000))
  assert set(perm[-3:].tolist()) == {0, 1, 2}
  p = perm[:-3]
  xyz = np.stack([np.cos(np.deg2rad(lat[p])) * np.cos(np.deg2rad(lon[p])),
                  np.cos(np.deg2rad(lat[p])) * np.sin(np.deg2rad(lon[p])), np.sin(np.deg2rad(lat[p]))], -1)
  step = np.linalg.norm(np.diff(xyz, axis=0), axis=1).mean()
  rand = np.linalg.norm(xyz[rng.permutation(len(p))] - xyz, axis=1).mean()
  assert step < 0.2 * rand


@pytest.mark.parametrize("n,bq,bk", [(100, 128, 128), (257, 128, 128), (1000, 128, 128), (300, 64, 32)])
def test_tile_mask_roundtrip(n, bq, bk):
  m = _random_mask(n, 0.05, 0)
  ptr, kb, bits = tiles.build_tile_mask(m, bq, bk)
  assert ptr[0] == 0 and ptr[-1] == len(kb) == len(bits)
  assert bits.shape[1:] == (bq, bk // 32)
  np.testing.assert_array_equal(tiles.tiles_to_dense(ptr, kb, bits, n, n, bq, bk), m.toarray())
  for qb in range(len(ptr) - 1):
    seg = kb[ptr[qb]:ptr[qb + 1]]
    assert len(np.unique(seg)) == len(seg) and (np.diff(seg) > 0).all()
    assert bits[ptr[qb]:ptr[qb + 1]].reshape(len(seg), -1).any(axis=1).all()


def test_sampled_attention_equals_dense():
  rng = np.random.default_rng(16)
  b, n, h, d = 2, 150, 3, 8
  q, k, v, do = (rng.standard_normal((b, n, h, d)) for _ in range(4))
  m = _random_mask(n, 0.06, 9)  # non-symmetric: dk/dv need the transposed neighbourhoods
  rows = np.array([0, 7, 149, 77])
  keys = np.array([3, 149, 0])
  got = A.sampled_attention(q, k, v, do, m, 0.3, rows, keys)
  out = A.dense_attention(q, k, v, m.toarray(), 0.3)
  lse = A.dense_lse(q, k, m.toarray(), 0.3)
  dq, dk, dv = A.dense_grads(q, k, v, do, m.toarray(), 0.3)
  np.testing.assert_allclose(got["out"], out[:, rows], atol=1e-12)
  np.testing.assert_allclose(got["lse"], lse[:, :, rows], atol=1e-12)
  np.testing.assert_allclose(got["dq"], dq[:, rows], atol=1e-12)
  np.testing.assert_allclose(got["dk"], dk[:, keys], atol=1e-12)
  np.testing.assert_allclose(got["dv"], dv[:, keys], atol=1e-12)


@pytest.mark.parametrize("symmetric", [True, False])
def test_block_attention_equals_dense(symmetric):
  """Whole 16-row/16-key blocks (block=16 keeps the dense check small) of a ragged n, with key blocks
  given out of order, a key block that no query reaches except through itself, and a row with no
  valid key (zero output and gradients, the kernels' convention)."""
  rng = np.random.default_rng(17)
  b, n, h, d, blk = 2, 90, 2, 8, 16
  q, k, v, do = (rng.standard_normal((b, n, h, d)) for _ in range(4))
  m = _random_mask(n, 0.05, 10, symmetric=symmetric).tolil()
  m[33, :] = False  # row 33 attends to nothing
  m = m.tocsr()
  dense = m.toarray()
  row_blocks, key_blocks = [5, 0, 2], [5, 1, 3]  # 5 is the ragged last block (rows 80-89)
  got = A.block_attention(q, k, v, do, m, 0.3, row_blocks, key_blocks, block=blk)
  rows = np.concatenate([np.arange(r * blk, min(n, (r + 1) * blk)) for r in row_blocks])
  keys = np.concatenate([np.arange(c * blk, min(n, (c + 1) * blk)) for c in key_blocks])
  np.testing.assert_array_equal(got["rows"], rows)
  np.testing.assert_array_equal(got["keys"], keys)
  live = dense.any(1)
  safe = dense | ~live[:, None]  # dense_* need every row to hold a key
  out = A.dense_attention(q, k, v, safe, 0.3) * live[None, :, None, None]
  lse = A.dense_lse(q, k, safe, 0.3)
  dq, dk, dv = A.dense_grads(q, k, v, do * live[None, :, None, None], safe, 0.3)
  dq = dq * live[None, :, None, None]
  np.testing.assert_allclose(got["out"], out[:, rows], atol=1e-12)
  np.testing.assert_allclose(got["lse"][:, :, live[rows]], lse[:, :, rows[live[rows]]], atol=1e-12)
  np.testing.assert_allclose(got["dq"], dq[:, rows], atol=1e-12)
  np.testing.assert_allclose(got["dk"], dk[:, keys], atol=1e-12)
  np.testing.assert_allclose(got["dv"], dv[:, keys], atol=1e-12)
  assert np.abs(got["out"][:, list(rows).index(33)]).max() == 0.0


# ---- oracle.rows: the gather/scatter either side of the layer loop and the layer norm ----

def test_rows_scatter_inverts_gather():
  rng = np.random.default_rng(0)
  x = rng.standard_normal((2, 50, 24))
  perm = rng.permutation(50)
  np.testing.assert_array_equal(rows.scatter(rows.gather(x, perm), perm), x)
  np.testing.assert_array_equal(rows.gather(rows.scatter(x, perm), perm), x)
  np.testing.assert_array_equal(rows.gather(x, np.arange(50)), x)
  # scatter with perm is take(., argsort(perm)) (patch.py:291-292)
  np.testing.assert_array_equal(rows.scatter(x, perm), np.take(x, np.argsort(perm), axis=1))


def test_rows_layer_norm_closed_forms():
  rng = np.random.default_rng(1)
  x = rng.standard_normal((3, 7, 40)) * 5 + 2
  eps = 1e-5
  y = rows.layer_norm(x, eps)
  var = x.var(-1)
  np.testing.assert_allclose(y.mean(-1), 0, atol=1e-12)
  np.testing.assert_allclose(y.var(-1), var / (var + eps), rtol=1e-12)
  # shift invariance, and scale invariance at eps = 0
  np.testing.assert_allclose(rows.layer_norm(x + 3.5, eps), y, atol=1e-12)
  np.testing.assert_allclose(rows.layer_norm(4 * x, 0.0), rows.layer_norm(x, 0.0), atol=1e-12)
  # a row of equally many a's and b's normalises to -1 / +1 (eps = 0)
  two = np.array([[[1.0, 3.0] * 8]])
  np.testing.assert_allclose(rows.layer_norm(two, 0.0), [[[-1.0, 1.0] * 8]], atol=1e-15)
  # a constant row has zero variance and normalises to 0
  np.testing.assert_array_equal(rows.layer_norm(np.full((1, 1, 8), 2.0), eps), 0.0)
  # the affine is applied per (batch, channel)
  mul, add = rng.standard_normal((3, 40)), rng.standard_normal((3, 40))
  np.testing.assert_allclose(rows.norm_affine(x, mul, add, eps), y * mul[:, None] + add[:, None], rtol=1e-15)
