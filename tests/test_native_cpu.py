"""CPU tests of the native library: exports, host mask pipeline vs the oracle, tile-list
preparation, argument validation, and the Python switch. No GPU is touched."""
import ctypes
import os
import re

import numpy as np
import pytest
from scipy import sparse

import faster_weathernext_amd as fwn
from faster_weathernext_amd import _native as nat
import hilbert_cases as HC
from oracle import mesh as om
from oracle import tiles as ot

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _random_mask(n, density, seed, symmetric=False):
  m = sparse.random(n, n, density=density, random_state=seed, format="csr").astype(bool)
  if symmetric:
    m = m + m.T
  return (m + sparse.identity(n, dtype=bool, format="csr")).tocsr().astype(bool)


def test_library_exports_every_declared_symbol():
  header = "".join(open(os.path.join(ROOT, "include", h)).read() for h in ("fwn_attn.h", "fwn_rows.h"))
  declared = set(re.findall(r"^(?:int|const char\*)\s+(fwn_\w+)\(", header, re.M))
  assert declared == set(nat.SIGNATURES), declared ^ set(nat.SIGNATURES)
  lib = ctypes.CDLL(nat.LIB_PATH)
  for name in declared:
    assert hasattr(lib, name), name
  assert nat.lib().fwn_last_error() is not None


@pytest.mark.parametrize("r", [0, 2, 4, 6])
def test_mesh_matches_oracle(r):
  v, f, lat, lon = fwn.icosahedral_mesh(r)
  v2, f2, lat2, lon2 = om.icosahedral_mesh(r)
  np.testing.assert_array_equal(f, f2)
  np.testing.assert_allclose(v, v2, rtol=0, atol=1e-15)
  np.testing.assert_allclose(lat, lat2, rtol=0, atol=1e-12)


@pytest.mark.parametrize("r,k", [(2, 0), (2, 1), (3, 2), (3, 5), (4, 8)])
def test_khop_matches_oracle(r, k):
  v, f, _, _ = om.icosahedral_mesh(r)
  adj = om.adjacency(f, len(v))
  got = fwn.khop_mask(adj, k)
  ref = om.khop_mask(adj, k)
  np.testing.assert_array_equal(got.indptr, ref.indptr)
  np.testing.assert_array_equal(got.indices, ref.indices)


def test_khop_r6_32hop_reference_keys_per_query():
  # docs/results/attn_bwd/attn_bwd_default_rtx5090.txt:3 of the reference: "3101 keys/query" for the
  # 32-hop mask of the 40,962-node mesh (independent of vertex numbering and orientation).
  mask, lat, lon, perm = fwn.mesh_mask(6, 32, reorder=True)
  n = mask.shape[0]
  assert n == 40962
  assert f"{mask.nnz / n:.0f}" == "3101"
  # Same log, line 4: "hilbert tiles: 5480 keys/query-block" at the reference's 64 x 32 tiles. It
  # depends on the exact vertex coordinates (the official mesh is not available here), so it is
  # matched to 0.1 %.
  inv = np.empty(n, np.int64)
  inv[perm] = np.arange(n)
  coo = mask.tocoo()
  qb, kb = inv[coo.row] // 64, inv[coo.col] // 32
  n_qb, n_kb = -(-n // 64), -(-n // 32)
  tiles = np.count_nonzero(np.bincount(qb * n_kb + kb, minlength=n_qb * n_kb))
  assert abs(tiles * 32 / n_qb - 5480) / 5480 < 1e-3


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_hilbert_octant_centres_follow_gray_code(seed):
  # Known answer from the mathematics of Skilling's transform and the reference's xyz convention
  # (tests/hilbert_cases.py): the eight octant centres in reflected Gray-code order, x leading.
  lat, lon, want = HC.octant_case(seed)
  np.testing.assert_array_equal(fwn.hilbert_order(lat, lon), want)


def test_hilbert_axis_points_quantise_to_the_formula_cells():
  # +-1 -> 0 / 1023 and 0 -> 511.5 rounded half to even (512), so -x, -z, {+x, +y, +z}, -y.
  names = list(HC.AXIS_POINTS)
  lat, lon = np.array([HC.AXIS_POINTS[k] for k in names]).T
  assert HC.axis_order_ok(fwn.hilbert_order(lat, lon), names)


def test_hilbert_matches_oracle():
  rng = np.random.default_rng(3)
  lat, lon = rng.uniform(-90, 90, 20000), rng.uniform(-180, 360, 20000)
  lat[[5, 17]] = np.nan
  lon[99] = np.inf
  got = fwn.hilbert_order(lat, lon)
  np.testing.assert_array_equal(got, ot.hilbert_order(lat, lon))
  assert set(got[-3:].tolist()) == {5, 17, 99}
  for bits in (1, 3, 16):
    np.testing.assert_array_equal(fwn.hilbert_order(lat, lon, bits), ot.hilbert_order(lat, lon, bits))


@pytest.mark.parametrize("n,density,permute", [(100, 0.05, False), (300, 0.08, True), (1000, 0.01, True),
                                               (129, 0.5, False)])
def test_tile_list_matches_oracle(n, density, permute):
  m = _random_mask(n, density, 7)
  perm = np.random.default_rng(1).permutation(n) if permute else None
  got = fwn.build_tile_mask(m, perm=perm)
  ref = ot.build_tile_mask(m[perm][:, perm] if permute else m, 128, 128)
  for g, r in zip(got, ref):
    np.testing.assert_array_equal(g, r)


def test_mask_without_valid_elements_has_no_tiles():
  """A mask with no valid element (and one of a single row) builds as the oracle does: every
  row block present in tile_ptr, no tiles (empty column and bit arrays); the schedule still has
  an item per block and the dS map no units."""
  for n in (1, 300):
    m = sparse.csr_matrix((n, n), dtype=bool)
    got = fwn.build_tile_mask(m)
    ref = ot.build_tile_mask(m, 128, 128)
    for g, r in zip(got, ref):
      np.testing.assert_array_equal(g, r)
    assert len(got[1]) == 0 and got[2].shape == (0, 128, 4)
    tl = fwn.TileList.from_mask(m, device="cpu")
    assert tl.n_tiles == 0 and tl.schedule_for(1, 2).n_items == -(-n // 128)
    status, ubase, tmap, n_units = _ds_map(got, got, 16)
    assert status == nat.OK and n_units == 0 and len(ubase) == 0 and len(tmap) == 0


def _decode_lanes(lanes, n_tiles):
  """Inverse of fwn_tiles_prepare's lane layout, written from the layout's definition."""
  bits = np.zeros((n_tiles, 128, 128), bool)
  lanes = lanes.reshape(n_tiles, 4, 64)  # tile, wave, lane; bit e = element e = (sub-block, register)
  for w in range(4):
    for lane in range(64):
      word = lanes[:, w, lane]
      row = 32 * w + (lane & 31)
      for sb in range(4):
        for r in range(16):
          col = 32 * sb + 16 * (r >> 3) + 8 * (lane >> 5) + (r & 7)
          bits[:, row, col] = (word >> np.uint64(16 * sb + r)) & np.uint64(1)
  return bits


def test_prepare_layout_roundtrip():
  n = 700
  m = _random_mask(n, 0.03, 11)
  m = m.tolil()
  m[0:128, 128:256] = True  # one fully valid tile
  m = m.tocsr()
  tp, kb, bits = fwn.build_tile_mask(m)
  T, nb = len(kb), len(tp) - 1
  lanes = np.zeros((T, nat.LANE_WORDS), np.uint64)
  groups = np.zeros(T, np.uint32)
  halves = np.zeros(T, np.uint32)
  nat.check(nat.lib().fwn_tiles_prepare(nb, T, n, nat.ptr(tp), nat.ptr(kb), nat.ptr(bits), nat.ptr(lanes),
                                        nat.ptr(groups), nat.ptr(halves)))
  dense = ((bits[:, :, :, None] >> np.arange(32, dtype=np.uint32)) & 1).astype(bool).reshape(T, 128, 128)
  np.testing.assert_array_equal(_decode_lanes(lanes, T), dense)
  # halves: bit 8r + 2c + h set iff rows 32r.. have a valid element in columns 32c + 16h .. +15.
  want = np.zeros(T, np.uint32)
  for r in range(4):
    for c in range(4):
      for h in range(2):
        blk = dense[:, 32 * r:32 * r + 32, 32 * c + 16 * h:32 * c + 16 * h + 16].reshape(T, -1)
        want |= blk.any(1).astype(np.uint32) << (8 * r + 2 * c + h)
  np.testing.assert_array_equal(halves, want)
  assert 0 < np.mean(halves != 0xFFFFFFFF)
  # a live group has at least one live half, a dead group none
  for r in range(4):
    for c in range(4):
      live = (groups >> (4 * r + c)) & 1
      hv = (halves >> (8 * r + 2 * c)) & 3
      np.testing.assert_array_equal(live.astype(bool), hv != 0)
  # groups: bit 4r + c set iff the 32 x 32 block (rows 32r.., columns 32c..) has a valid element,
  # bit 16 + 4r + c iff every element of it is valid.
  expect = np.zeros(T, np.uint32)
  for r in range(4):
    for c in range(4):
      blk = dense[:, 32 * r:32 * r + 32, 32 * c:32 * c + 32].reshape(T, -1)
      expect |= blk.any(1).astype(np.uint32) << (4 * r + c)
      expect |= blk.all(1).astype(np.uint32) << (16 + 4 * r + c)
  np.testing.assert_array_equal(groups, expect)
  full_tile = np.flatnonzero((tp[0] <= np.arange(T)) & (np.arange(T) < tp[1]) & (kb == 1))
  assert groups[full_tile[0]] == 0xFFFFFFFF
  assert 0 < np.mean((groups & 0xFFFF) != 0xFFFF)  # the random tiles leave some blocks empty
  assert np.all((groups >> 16) & ~groups & 0xFFFF == 0)  # full implies live


def test_prepare_groups_single_elements():
  # One valid element per tile at (row, column): exactly bit 4 * (row // 32) + column // 32.
  n = 512
  rows, cols = [5, 40, 70, 127, 300, 511], [100, 3, 64, 127, 33, 500]
  from scipy import sparse
  m = sparse.csr_matrix((np.ones(len(rows), bool), (rows, cols)), shape=(n, n))
  tp, kb, bits = fwn.build_tile_mask(m)
  T, nb = len(kb), len(tp) - 1
  lanes = np.zeros((T, nat.LANE_WORDS), np.uint64)
  groups = np.zeros(T, np.uint32)
  nat.check(nat.lib().fwn_tiles_prepare(nb, T, n, nat.ptr(tp), nat.ptr(kb), nat.ptr(bits), nat.ptr(lanes),
                                        nat.ptr(groups), None))
  got = {}
  for qb in range(nb):
    for t in range(tp[qb], tp[qb + 1]):
      got[(qb, int(kb[t]))] = int(groups[t])
  expect = {}
  for r, c in zip(rows, cols):
    key = (r // 128, c // 128)
    expect[key] = expect.get(key, 0) | 1 << (4 * ((r % 128) // 32) + (c % 128) // 32)
  assert got == expect


def _schedule(tp, max_item_tiles):
  L = nat.lib()
  nb = len(tp) - 1
  counts = np.zeros(3, np.int32)
  nat.check(L.fwn_tiles_schedule_count(nb, nat.ptr(tp), max_item_tiles, nat.ptr(counts[0:]), nat.ptr(counts[1:]),
                                       nat.ptr(counts[2:])))
  n_items, n_parts, n_split = (int(c) for c in counts)
  items = np.zeros((n_items, 4), np.int32)
  split = np.zeros((max(n_split, 1), 3), np.int32)
  nat.check(L.fwn_tiles_schedule_fill(nb, nat.ptr(tp), max_item_tiles, nat.ptr(items), nat.ptr(split)))
  return items, split[:n_split], n_parts


@pytest.mark.parametrize("max_item_tiles", [1, 2, 3, 7, 64, 0, -5])
def test_schedule_covers_every_tile_once(max_item_tiles):
  """Work items partition each block's tile run into near-equal pieces of at most max_item_tiles
  (default FWN_ITEM_TILES = 64 for max_item_tiles <= 0), in block order; split blocks own a
  contiguous range of partial slots."""
  rng = np.random.default_rng(3)
  counts = rng.integers(0, 200, 40)
  counts[[0, 5]] = 0  # empty blocks still get one item (they write zero rows)
  counts[7] = 320
  tp = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
  items, split, n_parts = _schedule(tp, max_item_tiles)
  cap = max_item_tiles if max_item_tiles > 0 else nat.ITEM_TILES
  lengths = items[:, 2] - items[:, 1]
  assert (np.diff(items[:, 0]) >= 0).all() and (np.diff(items[:, 1]) >= 0).all()
  assert lengths.max() <= max(cap, 0) or (lengths.max() == 0)
  covered = np.zeros(tp[-1], np.int32)
  for blk, t0, t1, part in items:
    assert tp[blk] <= t0 <= t1 <= tp[blk + 1]
    covered[t0:t1] += 1
  assert (covered == 1).all()
  per_block = np.bincount(items[:, 0], minlength=len(counts))
  assert (per_block == np.maximum(1, -(-counts // cap))).all()
  # Slots: whole blocks have part -1; split blocks' items use slots [first, first + count).
  whole = items[items[:, 3] < 0]
  assert (per_block[whole[:, 0]] == 1).all()
  assert sorted(items[items[:, 3] >= 0, 3].tolist()) == list(range(n_parts))
  for blk, first, cnt in split:
    mine = items[items[:, 0] == blk]
    assert sorted(mine[:, 3].tolist()) == list(range(first, first + cnt))
    ln = mine[:, 2] - mine[:, 1]
    assert ln.max() - ln.min() <= 1
  assert len(split) == int((per_block > 1).sum())
  assert n_parts == int(per_block[per_block > 1].sum())


ITEM_COST = 3  # the item cost these tests pass (tile costs of 1 when no per-tile costs are given)


def _order(items, pairs, order, window=0, tile_cost=None, item_cost=ITEM_COST, slots=32):
  L = nat.lib()
  n = np.zeros(1, np.int32)
  tc = nat.ptr(tile_cost) if tile_cost is not None else None
  nat.check(L.fwn_tiles_order_count(len(items), nat.ptr(items), tc, item_cost, pairs, order, window, slots,
                                    nat.ptr(n)))
  work = np.full((int(n[0]), 2), -7, np.int32)
  nat.check(L.fwn_tiles_order_fill(len(items), nat.ptr(items), tc, item_cost, pairs, order, window, slots,
                                   nat.ptr(work)))
  return work


def _makespan(costs, slots):
  """When the last job ends if `slots` slots take jobs of these durations in order (each to the
  first free slot): a brute-force event walk, independent of the library's heap."""
  free = [0] * slots
  end = 0
  for c in costs:
    s = min(range(slots), key=lambda i: (free[i], i))
    free[s] += c
    end = max(end, free[s])
  return end


def _xcd_jobs(work, n_items):
  """Per XCD (entry w runs on XCD w % 8), the jobs (pair * n_items + item) of its non-padding
  entries in launch order."""
  jobs = [[] for _ in range(8)]
  for w, (pair, item) in enumerate(work):
    if pair >= 0:
      jobs[w % 8].append(int(pair) * n_items + int(item))
  return jobs


@pytest.mark.parametrize("order,window", [(nat.ORDER_ITEMS, 0), (nat.ORDER_BALANCED, 0), (nat.ORDER_BALANCED, 1),
                                          (nat.ORDER_BALANCED, 7), (nat.ORDER_BALANCED, 128),
                                          (nat.ORDER_ITEMS, 32), (nat.ORDER_MAKESPAN, 0),
                                          (nat.ORDER_MAKESPAN, 64)])
@pytest.mark.parametrize("pairs", [1, 3, 8, 13])
def test_order_table_runs_every_job_once_in_contiguous_xcd_ranges(pairs, order, window):
  """An order table runs every (pair, item) job exactly once; XCD x (entries w = x mod 8) takes a
  contiguous range of the jobs in (pair, item) order, the ranges in XCD order; padding entries
  have pair -1. ITEMS: equal counts (without a window, the kernels' own mapping without a table,
  workgroup for workgroup). BALANCED: each range's cost (item cost 3 + tiles per job) is the
  even share total / 8 to within one job's cost. A window w > 1 sorts each consecutive w jobs of
  a range longest first (stable: ties in job order), counting the windows from the range's end so
  its last w jobs form one window; w <= 1 keeps job order."""
  rng = np.random.default_rng(pairs)
  counts = rng.integers(0, 200, 70)
  counts[:4] = 320  # long blocks first, as the subdivision order's coarse nodes
  tp = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
  items, _, _ = _schedule(tp, 64)
  ni = len(items)
  cost = ITEM_COST + items[:, 2] - items[:, 1]
  jcost = np.tile(cost, pairs)
  work = _order(items, pairs, order, window)
  total = ni * pairs
  assert len(work) % 8 == 0 and (work[:, 0] >= -1).all() and (work[:, 0] < pairs).all()
  assert ((work[:, 1] >= 0) & (work[:, 1] < ni)).all()
  assert (work[work[:, 0] < 0, 1] == 0).all()
  per = _xcd_jobs(work, ni)
  assert sorted(j for r in per for j in r) == list(range(total))
  starts = [min(r) if r else None for r in per]
  lo = 0
  for r in per:
    assert sorted(r) == list(range(lo, lo + len(r)))
    lo += len(r)
  # Every XCD's entries are its first len(r) slots (no padding between jobs).
  assert len(work) == 8 * max(len(r) for r in per)
  if order == nat.ORDER_ITEMS:
    small, rem = divmod(total, 8)
    assert [len(r) for r in per] == [small + (x < rem) for x in range(8)]
    assert len(work) == 8 * (small + (rem > 0))
  elif order == nat.ORDER_BALANCED:
    share = jcost.sum() / 8
    for r in per:
      assert abs(jcost[r].sum() - share) <= jcost.max()
  else:
    # no later end than the equal-cost cut's, simulated on the same 32 slots
    even = _xcd_jobs(_order(items, pairs, nat.ORDER_BALANCED, window), ni)
    assert max(_makespan(jcost[r], 32) for r in per) <= max(_makespan(jcost[r], 32) for r in even)
  if window <= 1:
    assert all(r == sorted(r) for r in per)
    if order == nat.ORDER_ITEMS:
      # the kernels' mapping without a table: workgroup 8 k + x runs the k-th job of XCD x
      for w in range(total):
        x, k = w % 8, w // 8
        job = x * (small + 1) + k if x < rem else rem * (small + 1) + (x - rem) * small + k
        assert tuple(work[w]) == (job // ni, job % ni)
  else:
    def windows(r):
      first = len(r) % window
      return ([r[:first]] if first else []) + [r[w0:w0 + window] for w0 in range(first, len(r), window)]
    for r in per:
      for win in windows(r):
        assert win == sorted(sorted(win), key=lambda j: -jcost[j])  # stable: ties in job order
    # each window holds the consecutive jobs at its positions of the (contiguous) range
    assert all([sorted(w) for w in windows(r)] == windows(sorted(r)) for r in per)


def test_order_table_known_answer():
  """Two pairs of five items, tiles 10, 0, 50, 4, 20 (costs 13, 3, 53, 7, 23 with item cost 3;
  198 for the ten jobs). A job goes to XCD floor(8 m / 198) for its cost midpoint m: midpoints
  6.5, 14.5, 42.5, 72.5, 87.5, 105.5, 113.5, 141.5, 171.5, 186.5 give XCDs 0, 0, 1, 2, 3, 4, 4,
  5, 6, 7. A plain split by count (ITEMS) gives two jobs to XCDs 0 and 1 and one to the rest."""
  lens = [10, 0, 50, 4, 20]
  t = np.concatenate([[0], np.cumsum(lens)])
  items = np.array([[b, t[b], t[b + 1], -1] for b in range(5)], np.int32)
  work = _order(items, 2, nat.ORDER_BALANCED)
  per = _xcd_jobs(work, 5)
  assert per == [[0, 1], [2], [3], [4], [5, 6], [7], [8], [9]]
  assert len(work) == 16 and tuple(work[8 + 4]) == (1, 1)  # XCD 4's second job: pair 1, item 1
  # windows of two: XCD 0 runs job 0 (13) before job 1 (3), XCD 4 job 5 (13) before 6 (3)
  assert _xcd_jobs(_order(items, 2, nat.ORDER_BALANCED, 2), 5) == per
  # windows counted from the end: five jobs of costs 4, 11, 4, 11, 4 (one XCD's worth) in windows
  # of two are [4], [11, 4], [11, 4] -> jobs 0, 1, 2, 3, 4; from the start they would be 1, 0, 3, 2, 4
  five = np.array([[0, 0, 1, -1], [1, 1, 9, -1]], np.int32)  # costs 4, 11
  assert _xcd_jobs(_order(five, 20, nat.ORDER_ITEMS, 2), 2)[0] == [0, 1, 2, 3, 4]
  lens2 = np.array([[0, 0, 1, -1], [1, 1, 9, -1]], np.int32)  # costs 4, 11: windows reorder
  assert _xcd_jobs(_order(lens2, 8, nat.ORDER_ITEMS, 2), 2) == [[1, 0], [3, 2], [5, 4], [7, 6], [9, 8],
                                                                  [11, 10], [13, 12], [15, 14]]
  per = _xcd_jobs(_order(items, 2, nat.ORDER_ITEMS, 4), 5)  # counts 2, 2, 1, 1, 1, 1, 1, 1
  assert per == [[0, 1], [2, 3], [4], [5], [6], [7], [8], [9]]
  per = _xcd_jobs(_order(items, 1, nat.ORDER_ITEMS, 0), 5)  # 5 jobs: XCDs 0-4 one each
  assert per == [[0], [1], [2], [3], [4], [], [], []]


def test_order_table_weighs_tiles_by_their_costs():
  """With per-tile costs an item costs item_cost plus its tiles' costs: two pairs of three items
  of tiles [0, 2), [2, 3), [3, 6) with tile costs 5, 5, 40, 1, 1, 1 and item cost 2 cost 12, 42,
  5 (118 in all). Midpoints 6, 33, 56.5, 65, 92, 115.5 give XCDs floor(8 m / 118) = 0, 2, 3, 4,
  6, 7. With tile costs of 1 (costs 4, 3, 5; 24 in all) the midpoints 2, 5.5, 9.5, 14, 17.5, 21.5
  give XCDs 0, 1, 3, 4, 5, 7."""
  items = np.array([[0, 0, 2, -1], [1, 2, 3, -1], [2, 3, 6, -1]], np.int32)
  tc = np.array([5, 5, 40, 1, 1, 1], np.int32)
  per = _xcd_jobs(_order(items, 2, nat.ORDER_BALANCED, 0, tc, 2), 3)
  assert per == [[0], [], [1], [2], [3], [], [4], [5]]
  per = _xcd_jobs(_order(items, 2, nat.ORDER_BALANCED, 0, None, 2), 3)
  assert per == [[0], [1], [], [2], [3], [4], [], [5]]


def test_makespan_cut_evens_the_last_rounds():
  """FWN_ORDER_MAKESPAN on 4 slots per XCD: four pairs of 24 items (tiles below, item cost 2).
  The equal-cost cut gives the XCDs 11 and 13 jobs in turn, and the latest simulated end (each
  job to the first free of 4 slots; `_makespan` walks it without the library) is 31. The makespan
  cut gives every XCD 12 jobs and ends at 30; no order it returns ends later than the equal-cost
  one (checked for every case in the test above)."""
  lens = [8, 11, 10, 6, 11, 11, 11, 1, 5, 7, 4, 5, 7, 9, 7, 2, 8, 10, 3, 6, 4, 10, 1, 6]
  t = np.concatenate([[0], np.cumsum(lens)])
  items = np.array([[b, t[b], t[b + 1], -1] for b in range(24)], np.int32)
  cost = np.tile(2 + np.array(lens), 4)
  even = _xcd_jobs(_order(items, 4, nat.ORDER_BALANCED, 0, None, 2), 24)
  cut = _xcd_jobs(_order(items, 4, nat.ORDER_MAKESPAN, 0, None, 2, slots=4), 24)
  assert [len(r) for r in even] == [11, 13] * 4 and [len(r) for r in cut] == [12] * 8
  assert sorted(j for r in cut for j in r) == list(range(96))
  assert max(_makespan(cost[r], 4) for r in even) == 31 and max(_makespan(cost[r], 4) for r in cut) == 30


def test_order_table_rejects_bad_arguments():
  L = nat.lib()
  items = np.array([[0, 0, 5, -1], [1, 5, 9, -1]], np.int32)
  n = np.zeros(1, np.int32)
  assert L.fwn_tiles_order_count(2, nat.ptr(items), None, 3, 2, 7, 0, 32, nat.ptr(n)) == nat.ERR_INVALID_ARG
  assert b"unknown order" in L.fwn_last_error()
  assert L.fwn_tiles_order_count(0, nat.ptr(items), None, 3, 2, 1, 0, 32, nat.ptr(n)) == nat.ERR_INVALID_ARG
  assert L.fwn_tiles_order_count(2, nat.ptr(items), None, 3, 0, 1, 0, 32, nat.ptr(n)) == nat.ERR_INVALID_ARG
  assert L.fwn_tiles_order_count(2, nat.ptr(items), None, -1, 2, 1, 0, 32, nat.ptr(n)) == nat.ERR_INVALID_ARG
  assert L.fwn_tiles_order_count(2, nat.ptr(items), None, 3, 2, nat.ORDER_MAKESPAN, 0, 0, nat.ptr(n)) \
      == nat.ERR_INVALID_ARG
  assert b"slots" in L.fwn_last_error()
  neg = np.ones(9, np.int32)
  neg[6] = -2
  assert L.fwn_tiles_order_count(2, nat.ptr(items), nat.ptr(neg), 3, 2, 1, 0, 32, nat.ptr(n)) == nat.ERR_INVALID_ARG
  assert b"negative cost" in L.fwn_last_error()
  bad = items.copy()
  bad[1, 2] = 4
  assert L.fwn_tiles_order_count(2, nat.ptr(bad), None, 3, 2, 1, 0, 32, nat.ptr(n)) == nat.ERR_TILES
  assert L.fwn_tiles_order_fill(2, nat.ptr(items), None, 3, 2, 1, 0, 32, None) == nat.ERR_INVALID_ARG


def test_tile_list_orders_calls_with_few_jobs():
  """Calls whose per-item launch has fewer than ORDER_JOBS jobs get the schedule's order table
  for their (batch, head) count and kernel, with the window ORDER_WINDOWS gives their products;
  calls with many jobs get none; the workspace does not depend on the table."""
  from faster_weathernext_amd import hip_attn
  mask, _, _, _ = fwn.mesh_mask(5, 4)
  tl = hip_attn.TileList.from_mask(mask, device="cpu")
  n = mask.shape[0]
  bf16 = nat.AttnDesc(1, n, 4, 64, nat.BF16, 0.1, 4 * 64, 4 * 64, 64)
  f32 = nat.AttnDesc(1, n, 4, 64, nat.F32, 0.1, 4 * 64, 4 * 64, 64)
  x3 = nat.AttnDesc(1, n, 4, 64, nat.F32, 0.1, 4 * 64, 4 * 64, 64, 0, 0, 0, nat.PREC_BF16X3, 0)
  sch = tl.schedule_for(1, 4)
  assert tl.order_for(1, 4)
  for desc, products in ((bf16, "bf16"), (f32, "f32"), (x3, "bf16x3")):
    for kernel in ("fwd", "dq", "kv"):
      plan = (hip_attn.ORDER_CUTS[kernel], hip_attn.ORDER_WINDOWS[products][kernel], hip_attn.ORDER_SLOTS[kernel])
      assert hip_attn.order_plan(desc, kernel) == plan
      st = tl.struct_for_desc(desc, kernel)
      table = tl.schedule_for(1, 4, kernel).order_table(4, *plan)
      assert st.work and st.work_pairs == 4 and st.n_work == len(table)
      assert tl.struct_for_desc(desc, kernel) is st  # built once
      size = ctypes.c_uint64(0)
      nat.check(nat.lib().fwn_attn_workspace_size(desc, st, ctypes.byref(size)))
      assert tl.workspace_bytes(desc) >= int(size.value)
  assert hip_attn.ORDER_WINDOWS["bf16"] == {"fwd": 64, "dq": 64, "kv": 32}
  # dK/dV's items are cut at WIDE_ITEM_TILES, the others at nat.ITEM_TILES below WIDE_JOBS; the
  # workspace is the largest any of the three needs
  assert tl.item_cap_for(1, 4, "kv") == hip_attn.WIDE_ITEM_TILES and tl.item_cap_for(1, 4) == nat.ITEM_TILES
  assert tl.struct_for_desc(bf16, "kv").n_items == tl.schedule_for(1, 4, "kv").n_items
  sizes = []
  for kernel in ("fwd", "dq", "kv"):
    size = ctypes.c_uint64(0)
    nat.check(nat.lib().fwn_attn_workspace_size(bf16, tl.schedule_for(1, 4, kernel).struct, ctypes.byref(size)))
    sizes.append(int(size.value))
  assert tl.workspace_bytes(bf16) == max(sizes)
  many = -(-hip_attn.ORDER_JOBS // (sch.n_items * 4))
  assert not tl.order_for(many, 4) and tl.struct_for(many, 4, (nat.ORDER_BALANCED, 128, 64)).n_work == 0


@pytest.mark.parametrize("case", ["pairs", "short", "no_table"])
def test_launchers_reject_order_tables_that_do_not_fit_the_call(case):
  tiles = _tiles()  # 3 items
  if case == "pairs":
    tiles.work, tiles.n_work, tiles.work_pairs = FAKE, 48, 1
  elif case == "short":
    tiles.work, tiles.n_work, tiles.work_pairs = FAKE, 5, 2
  else:
    tiles.n_work = 8
  size = ctypes.c_uint64(0)
  assert nat.lib().fwn_attn_workspace_size(_desc(n=300), tiles, ctypes.byref(size)) == nat.ERR_TILES  # heads 2
  assert b"order table" in nat.lib().fwn_last_error()


@pytest.mark.parametrize("case", ["ptr0", "decreasing", "col_range", "col_order", "total", "tail_bits"])
def test_prepare_rejects_malformed_lists(case):
  n = 300
  tp, kb, bits = fwn.build_tile_mask(_random_mask(n, 0.05, 2))
  tp, kb, bits = tp.copy(), kb.copy(), bits.copy()
  if case == "ptr0":
    tp[0] = 1
  elif case == "decreasing":
    tp[1], tp[2] = tp[2], tp[1]
  elif case == "col_range":
    kb[0] = 3
  elif case == "col_order":
    kb[1] = kb[0]
  elif case == "total":
    tp[-1] -= 1
  elif case == "tail_bits":
    last = np.flatnonzero(kb == 2)[0]
    bits[last, 0, 3] |= np.uint32(1 << 31)  # column 2*128 + 127 >= n
  T, nb = len(kb), len(tp) - 1
  lanes = np.zeros((T, nat.LANE_WORDS), np.uint64)
  groups = np.zeros(T, np.uint32)
  status = nat.lib().fwn_tiles_prepare(nb, T, n, nat.ptr(tp), nat.ptr(kb), nat.ptr(bits), nat.ptr(lanes),
                                       nat.ptr(groups), None)
  assert status == nat.ERR_TILES
  assert nat.lib().fwn_last_error()


def _desc(**kw):
  d = dict(batch=1, n=300, heads=2, head_dim=64, dtype=nat.F32, scale=0.125, stride_b=300 * 128,
           stride_n=128, stride_h=64)
  d.update(kw)
  return nat.AttnDesc(**d)


FAKE = 1 << 20  # a device address the launchers never dereference: validation fails first


def _tiles(n_blocks=3, n_tiles=0, n_items=3, n_parts=0, n_split=0, ptr=FAKE, items=FAKE, split=None):
  return nat.Tiles(n_blocks, n_tiles, ptr, None, None, None, n_items, n_parts, n_split, 0, items, split)


@pytest.mark.parametrize("kw,code", [
    (dict(head_dim=48), nat.ERR_UNSUPPORTED), (dict(dtype=7), nat.ERR_UNSUPPORTED),
    (dict(n=0), nat.ERR_INVALID_ARG), (dict(scale=0.0), nat.ERR_INVALID_ARG),
    (dict(scale=float("nan")), nat.ERR_INVALID_ARG), (dict(stride_n=66), nat.ERR_INVALID_ARG),
    (dict(stride_n=32), nat.ERR_INVALID_ARG), (dict(n=40962, stride_n=1 << 16), nat.ERR_INVALID_ARG)])
def test_launchers_validate_before_launching(kw, code):
  # Every launcher checks its arguments on the host and returns before any HIP call.
  tiles = _tiles(ptr=None, items=None)
  desc = _desc(**kw)
  fake = FAKE
  L = nat.lib()
  assert L.fwn_attn_fwd_launch(desc, fake, fake, fake, tiles, fake, None, None, 0, None) == code
  assert L.fwn_attn_bwd_delta_launch(desc, fake, fake, fake, None) == code
  assert L.fwn_attn_bwd_dq_launch(desc, fake, fake, fake, fake, fake, fake, tiles, fake, None, 0, None) == code
  assert L.fwn_attn_bwd_dkv_launch(desc, fake, fake, fake, fake, fake, fake, tiles, fake, fake, None, 0, None) == code


def test_launchers_reject_bad_pointers_and_tiles():
  L = nat.lib()
  desc = _desc()
  F = FAKE
  good = _tiles()
  assert L.fwn_attn_fwd_launch(desc, None, F, F, good, F, None, None, 0, None) == nat.ERR_INVALID_ARG
  assert L.fwn_attn_fwd_launch(desc, F + 4, F, F, good, F, None, None, 0, None) == nat.ERR_INVALID_ARG
  assert L.fwn_attn_fwd_launch(desc, F, F, F, _tiles(n_blocks=5), F, None, None, 0, None) == nat.ERR_TILES
  assert L.fwn_attn_fwd_launch(desc, F, F, F, _tiles(n_tiles=10), F, None, None, 0, None) == nat.ERR_TILES
  assert "tiles" in L.fwn_last_error().decode()
  # every block needs a work item; split schedules need their slot table
  assert L.fwn_attn_fwd_launch(desc, F, F, F, _tiles(n_items=2), F, None, None, 0, None) == nat.ERR_TILES
  assert L.fwn_attn_fwd_launch(desc, F, F, F, _tiles(items=None), F, None, None, 0, None) == nat.ERR_TILES
  assert L.fwn_attn_fwd_launch(desc, F, F, F, _tiles(n_items=4, n_parts=2, n_split=1), F, None, None, 0,
                               None) == nat.ERR_TILES
  assert L.fwn_attn_fwd_launch(desc, F, F, F, _tiles(n_items=4, n_parts=2), F, None, None, 0, None) == nat.ERR_TILES


def test_output_strides_are_validated_separately():
  """o/dout strides (ostride_*) are checked like the q/k/v strides; all zero means 'the same'."""
  L = nat.lib()
  F = FAKE
  good = _tiles()
  packed = _desc(stride_b=300 * 3 * 2 * 64, stride_n=3 * 2 * 64, stride_h=64)  # q, k, v views of [B, n, 3, H, D]
  assert L.fwn_attn_fwd_launch(packed, F, F, F, _tiles(n_blocks=5), F, None, None, 0, None) == nat.ERR_TILES
  for bad in (dict(ostride_b=300 * 128, ostride_n=66, ostride_h=64),      # not a multiple of 16 bytes
              dict(ostride_b=300 * 128, ostride_n=32, ostride_h=64),      # rows overlap
              dict(ostride_b=0, ostride_n=1 << 21, ostride_h=64)):        # slice beyond 2 GiB offsets
    d = _desc(**bad)
    assert L.fwn_attn_fwd_launch(d, F, F, F, good, F, None, None, 0, None) == nat.ERR_INVALID_ARG
    assert "o/dout" in L.fwn_last_error().decode()
    assert L.fwn_attn_bwd_delta_launch(d, F, F, F, None) == nat.ERR_INVALID_ARG


def test_workspace_size_and_checks():
  """Split schedules need n_parts * batch * heads * 128 * (2 * head_dim + 2) * 4 bytes of
  256-byte-aligned workspace; launchers refuse a missing, short or misaligned one."""
  import ctypes
  L = nat.lib()
  F = FAKE
  desc = _desc(batch=2, heads=3, head_dim=64, stride_b=300 * 3 * 64, stride_n=3 * 64, stride_h=64)
  split = _tiles(n_items=5, n_parts=3, n_split=1, split=F)
  size = ctypes.c_uint64(0)
  nat.check(L.fwn_attn_workspace_size(desc, split, ctypes.byref(size)))
  need = 3 * 2 * 3 * 128 * (2 * 64 + 2) * 4
  assert size.value == need
  nat.check(L.fwn_attn_workspace_size(desc, _tiles(), ctypes.byref(size)))
  assert size.value == 0
  for ws, nbytes in [(None, need), (F + 16, need), (F, need - 1)]:
    assert L.fwn_attn_fwd_launch(desc, F, F, F, split, F, None, ws, nbytes, None) == nat.ERR_INVALID_ARG
    assert L.fwn_attn_bwd_dq_launch(desc, F, F, F, F, F, F, split, F, ws, nbytes, None) == nat.ERR_INVALID_ARG
    assert L.fwn_attn_bwd_dkv_launch(desc, F, F, F, F, F, F, split, F, F, ws, nbytes, None) == nat.ERR_INVALID_ARG
    assert "workspace" in L.fwn_last_error().decode()


def test_enable_disable_and_unknown_option():
  # tests/test_masks.py:91-102 of the reference: enable/disable round trip, unknown option raises.
  import torch
  from faster_weathernext_amd import patch
  # Without a gfx950 (this host has no GPU) enable() refuses, as attention_impl() does, and leaves
  # the options unchanged; force skips the check, as the reference's force skips its compat check.
  if patch.device_arch() != patch.ARCH:
    with pytest.raises(RuntimeError, match="gfx950"):
      fwn.enable(reorder=False)
    with pytest.raises(RuntimeError, match="gfx950"):
      patch.attention_impl()
    assert not patch.is_enabled() and fwn.options().reorder is True
  opts = fwn.enable(force=True, reorder=False, bf16=True)
  assert patch.is_enabled() and opts.reorder is False and opts.bf16 is True
  # The options are the defaults of the modules built afterwards.
  assert patch.default_reorder() is False and patch.default_reorder(True) is True
  assert patch.default_dtype() is torch.bfloat16 and patch.default_dtype(torch.float32) is torch.float32
  mha = fwn.TiledMHA(16, 2, 8, None, device="cpu")
  assert mha.qkv.weight.dtype is torch.bfloat16
  fwn.disable()
  assert not patch.is_enabled() and fwn.options().reorder is True and patch.default_dtype() is torch.float32
  assert fwn.TiledMHA(16, 2, 8, None, device="cpu").qkv.weight.dtype is torch.float32
  with pytest.raises(TypeError):
    fwn.enable(not_an_option=1)
  with pytest.raises(ValueError):
    fwn.enable(force=True, attention="pallas")
  assert not patch.is_enabled()
  fwn.disable()


def test_khop_of_a_directed_adjacency_is_the_boolean_power():
  """Row i of the k-hop mask is row i of (adj + I)^k also when adj is not symmetric."""
  n, k = 300, 3
  adj = sparse.random(n, n, density=0.01, random_state=7, format="csr").astype(bool)
  assert (adj != adj.T).nnz
  power = sparse.identity(n, dtype=np.int64, format="csr")
  step = (adj + sparse.identity(n, dtype=bool, format="csr")).astype(np.int64)
  for _ in range(k):
    power = ((power @ step) > 0).astype(np.int64)
  got = fwn.khop_mask(adj, k)
  np.testing.assert_array_equal(got.toarray(), power.toarray() > 0)


def test_mesh_transformer_builds_the_transposed_list_for_a_directed_adjacency():
  """MeshTransformer on a caller's adjacency (patch.py:193-219): a non-symmetric adjacency gets the
  transposed mask's tile list (of the Hilbert-permuted mask) for the backward, shared by every
  block; a symmetric one gets none."""
  v, f, lat, lon = fwn.icosahedral_mesh(2)
  n = len(v)
  sym = fwn.adjacency(f, n)
  rng = np.random.default_rng(3)
  keep = rng.random(sym.nnz) < 0.7  # drop 30% of the directed edges: no longer symmetric
  coo = sym.tocoo()
  directed = sparse.csr_matrix((np.ones(int(keep.sum()), bool), (coo.row[keep], coo.col[keep])), shape=(n, n))
  kw = dict(k_hop=2, num_layers=2, d_model=16, num_heads=2, key_size=32, ffw_hidden=32, cond_size=4, device="cpu")
  model = fwn.MeshTransformer(adjacency=directed, latlon=(lat, lon), reorder=True, **kw)
  assert model.tiles_t is not None and all(b.mha.tiles_t is model.tiles_t for b in model.blocks)
  perm = fwn.hilbert_order(lat, lon)
  mask = fwn.khop_mask(directed, 2)[perm][:, perm]
  want = fwn.build_tile_mask(mask.T.tocsr())
  assert model.tiles_t.n_tiles == len(want[1])
  np.testing.assert_array_equal(model.tiles_t.col.numpy(), want[1])
  np.testing.assert_array_equal(model.perm.numpy(), perm)
  assert fwn.MeshTransformer(adjacency=sym, latlon=(lat, lon), reorder=True, **kw).tiles_t is None
  assert fwn.MeshTransformer(refinement=2, reorder=False, **kw).tiles_t is None


def test_public_op_refuses_cpu_tensors():
  import torch
  q = torch.zeros(1, 10, 1, 32)
  tp, kb, bits = fwn.build_tile_mask(sparse.identity(10, dtype=bool, format="csr"))
  with pytest.raises(ValueError, match="GPU"):
    fwn.tiled_flash_attention(q, q, q, tp, kb, bits, scale=1.0)


def test_tile_cache_round_trip_and_invalidation(tmp_path):
  """The cache returns the built tile list bit for bit on a hit; another k, a changed adjacency, a
  corrupt or truncated file are misses and are rebuilt."""
  from faster_weathernext_amd import tile_cache
  v, f, lat, lon = fwn.icosahedral_mesh(3)
  adj = fwn.adjacency(f, len(v))
  perm = fwn.hilbert_order(lat, lon)
  ref = fwn.build_tile_mask(fwn.khop_mask(adj, 2), perm=perm)
  got = tile_cache.cached_khop_tiles(adj, 2, perm, cache_dir=str(tmp_path))
  assert not got[3]
  for a, b in zip(got[:3], ref):
    np.testing.assert_array_equal(a, b)
  hit = tile_cache.cached_khop_tiles(adj, 2, perm, cache_dir=str(tmp_path))
  assert hit[3]
  for a, b in zip(hit[:3], ref):
    np.testing.assert_array_equal(a, b)
  assert not tile_cache.cached_khop_tiles(adj, 3, perm, cache_dir=str(tmp_path))[3]   # other k
  assert not tile_cache.cached_khop_tiles(adj, 2, None, cache_dir=str(tmp_path))[3]   # other order
  (path,) = [p for p in tmp_path.iterdir() if p.name.startswith("khop2_") and
             p.name.endswith(f"{tile_cache.mask_key(adj, perm, 2):016x}.fwnt")]
  raw = path.read_bytes()
  path.write_bytes(raw[:-4])                                                          # truncated
  assert not tile_cache.cached_khop_tiles(adj, 2, perm, cache_dir=str(tmp_path))[3]
  bad = bytearray(path.read_bytes())
  bad[0:8] = b"XXXXXXXX"                                                               # wrong magic
  path.write_bytes(bytes(bad))
  assert not tile_cache.cached_khop_tiles(adj, 2, perm, cache_dir=str(tmp_path))[3]
  assert tile_cache.cached_khop_tiles(adj, 2, perm, cache_dir=str(tmp_path))[3]
  # header fields as documented
  head = tile_cache._HEADER.unpack_from(path.read_bytes())
  assert head[0] == b"FWNTILES" and head[1] == 1 and head[2] == head[3] == len(v) and head[4] == 2 and head[5] == 1
  assert head[6] == 128 and head[8] == len(ref[0]) - 1 and head[9] == len(ref[1])


def test_tile_mask_cache_keys_on_content(tmp_path):
  from faster_weathernext_amd import tile_cache
  m = _random_mask(400, 0.03, 7)
  a = tile_cache.cached_tile_mask(m, cache_dir=str(tmp_path))
  assert not a[3] and tile_cache.cached_tile_mask(m, cache_dir=str(tmp_path))[3]
  m2 = m.tolil()
  m2[0, 399] = not m2[0, 399]
  b = tile_cache.cached_tile_mask(m2.tocsr(), cache_dir=str(tmp_path))
  assert not b[3]
  ref = fwn.build_tile_mask(m2.tocsr())
  for x, y in zip(b[:3], ref):
    np.testing.assert_array_equal(x, y)


# ---- row permutation passes (include/fwn_rows.h): host validation, no GPU calls ----

_ROW_PTR = 1 << 20  # an aligned fake device address: validation fails before any launch


def _rows_desc(**kw):
  d = dict(batch=1, n=64, channels=768, dtype=nat.F32, eps=1e-5)
  d.update(kw)
  return nat.RowsDesc(d["batch"], d["n"], d["channels"], d["dtype"], d["eps"])


@pytest.mark.parametrize("kw, code", [
    (dict(channels=0), nat.ERR_INVALID_ARG),
    (dict(channels=12), nat.ERR_INVALID_ARG),                 # not a multiple of 8
    (dict(channels=nat.ROWS_MAX_CHANNELS + 8), nat.ERR_INVALID_ARG),
    (dict(n=-1), nat.ERR_INVALID_ARG),
    (dict(batch=-2), nat.ERR_INVALID_ARG),
    (dict(dtype=7), nat.ERR_UNSUPPORTED),
    (dict(eps=float("nan")), nat.ERR_INVALID_ARG),
    (dict(eps=-1.0), nat.ERR_INVALID_ARG),
])
def test_rows_launchers_reject_bad_descriptors(kw, code):
  L = nat.lib()
  d = _rows_desc(**kw)
  P = _ROW_PTR
  assert L.fwn_rows_gather_norm_launch(d, P, P + (1 << 24), P + (2 << 24), P + (3 << 24), None) == code
  assert L.fwn_rows_norm_scatter_launch(d, P, P + (1 << 24), None, None, P + (2 << 24), None) == code
  assert L.fwn_rows_norm_affine_launch(d, P, None, None, P + (2 << 24), None) == code
  assert L.fwn_rows_add_norm_affine_launch(d, P, P + (1 << 24), None, None, P + (3 << 24), P + (2 << 24), None) == code
  assert L.fwn_last_error()


def test_rows_launchers_reject_bad_pointers():
  L = nat.lib()
  d = _rows_desc()
  P, Q, R, S = _ROW_PTR, _ROW_PTR + (1 << 24), _ROW_PTR + (2 << 24), _ROW_PTR + (3 << 24)
  bad = nat.ERR_INVALID_ARG
  assert L.fwn_rows_gather_norm_launch(None, P, Q, R, S, None) == bad
  assert L.fwn_rows_gather_norm_launch(d, None, Q, R, S, None) == bad   # x
  assert L.fwn_rows_gather_norm_launch(d, P, None, R, S, None) == bad   # perm
  assert L.fwn_rows_gather_norm_launch(d, P, Q, None, S, None) == bad   # x_out
  assert L.fwn_rows_gather_norm_launch(d, P + 4, Q, R, S, None) == bad  # misaligned x
  assert L.fwn_rows_gather_norm_launch(d, P, Q, R, S + 8, None) == bad  # misaligned norm_out
  assert L.fwn_rows_gather_norm_launch(d, P, Q, P + 64, S, None) == bad  # x_out overlaps x
  assert L.fwn_rows_gather_norm_launch(d, P, Q, R, R + 64, None) == bad  # norm_out overlaps x_out
  assert L.fwn_rows_norm_scatter_launch(d, P, Q, None, None, None, None) == bad  # out
  assert L.fwn_rows_norm_scatter_launch(d, P, Q, R + 4, None, S, None) == bad    # misaligned mul
  assert L.fwn_rows_norm_scatter_launch(d, P, Q, None, R + 4, S, None) == bad    # misaligned add
  assert L.fwn_rows_norm_scatter_launch(d, P, Q, None, None, P + 64, None) == bad  # out overlaps x
  assert L.fwn_rows_norm_affine_launch(d, None, None, None, S, None) == bad     # x
  assert L.fwn_rows_norm_affine_launch(d, P, None, None, None, None) == bad     # out
  assert L.fwn_rows_norm_affine_launch(d, P, R + 4, None, S, None) == bad       # misaligned mul
  assert L.fwn_rows_norm_affine_launch(d, P, None, R + 4, S, None) == bad       # misaligned add
  assert L.fwn_rows_norm_affine_launch(d, P, None, None, P + 64, None) == bad   # out overlaps x
  assert b"overlap" in L.fwn_last_error()
  add_norm = L.fwn_rows_add_norm_affine_launch  # (d, x, y, mul, add, sum, out, stream)
  assert add_norm(d, P, None, None, None, R, S, None) == bad        # y
  assert add_norm(d, P, Q, None, None, None, S, None) == bad        # sum
  assert add_norm(d, P, Q, None, None, R, None, None) == bad        # out
  assert add_norm(d, P, Q + 4, None, None, R, S, None) == bad       # misaligned y
  assert add_norm(d, P, Q, R + 4, None, R, S, None) == bad          # misaligned mul
  assert add_norm(d, P, Q, None, None, R, Q + 64, None) == bad      # out overlaps y
  assert add_norm(d, P, Q, None, None, S, S, None) == bad           # out overlaps sum
  assert add_norm(d, P, Q, None, None, P + 64, S, None) == bad      # sum shifted against x
  assert add_norm(d, P, Q, None, None, Q + 64, S, None) == bad      # sum shifted against y
  assert b"sum must be x, y or disjoint" in L.fwn_last_error()


def test_rows_python_wrappers_reject_cpu_tensors():
  import torch
  from faster_weathernext_amd import rows
  x = torch.zeros(1, 16, 64)
  perm = torch.arange(16)
  with pytest.raises(ValueError):
    rows.gather_layer_norm(x, perm)
  with pytest.raises(ValueError):
    rows.layer_norm_scatter(x, perm)


def test_tile_list_picks_the_split_schedule_per_launch():
  """With no cap given, a TileList launches short items (nat.ITEM_TILES) for few jobs and long
  ones (WIDE_ITEM_TILES) from WIDE_JOBS = blocks x batch x heads up; a given cap is always used."""
  from faster_weathernext_amd import hip_attn
  nb = 130  # block 0 has all 130 column tiles (3 items at cap 64, 2 at 128), the others their diagonal
  tp = np.concatenate([[0], nb + np.arange(nb, dtype=np.int32)]).astype(np.int32)
  kb = np.concatenate([np.arange(nb), np.arange(1, nb)]).astype(np.int32)
  bits = np.full((len(kb), nat.BLOCK, nat.BLOCK // 32), 0xFFFFFFFF, np.uint32)
  n = nb * nat.BLOCK
  tl = hip_attn.TileList(tp, kb, bits, n, device="cpu")
  assert tl.struct.n_items == tl.n_items == nb + 2 and tl.struct.n_parts == 3
  jobs = -(-hip_attn.WIDE_JOBS // nb)  # batch members that reach WIDE_JOBS with one head
  assert tl.struct_for(jobs - 1, 1).n_items == nb + 2
  wide = tl.struct_for(jobs, 1)
  assert wide.n_items == nb + 1 and wide.n_parts == 2
  assert tl.struct_for(jobs, 1) is wide  # built once
  fixed = hip_attn.TileList(tp, kb, bits, n, device="cpu", max_item_tiles=32)
  assert fixed.struct_for(8, 64).n_items == fixed.struct.n_items == nb + 4
  assert tl.schedule_for(jobs, 1).struct is wide and tl.item_cap_for(jobs, 1) == hip_attn.WIDE_ITEM_TILES
  assert list(tl.schedule_for(jobs, 1).split_host[:, 0]) == [0]  # block 0 is the one split block
  # The workspace is sized for the schedule the call launches, not for the 64-tile one.
  for batch, st in ((jobs, wide), (jobs - 1, tl.struct)):
    desc = nat.AttnDesc(batch, n, 1, 128, nat.BF16, 0.1, n * 128, 128, 128, n * 128, 128, 128)  # [batch, n, 1, 128]
    size = ctypes.c_uint64(0)
    nat.check(nat.lib().fwn_attn_workspace_size(desc, st, ctypes.byref(size)))
    assert tl.workspace_bytes(desc) == int(size.value) == st.n_parts * batch * 128 * (2 * 128 + 2) * 4
  # Nothing split: no workspace at all.
  diag = hip_attn.TileList(np.arange(nb + 1, dtype=np.int32), np.arange(nb, dtype=np.int32), bits[:nb], n,
                           device="cpu")
  assert diag.workspace_bytes(nat.AttnDesc(1, n, 1, 128, nat.BF16, 0.1, n * 128, 128, 128, 0, 0, 0)) == 0
  assert hip_attn.workspace(nat.AttnDesc(1, n, 1, 128, nat.BF16, 0.1, n * 128, 128, 128, 0, 0, 0), "cpu", diag) is None


def test_tile_lists_reject_foreign_formats_and_mismatched_calls():
  """The reference's 64 x 32 tile bits (uint32[T, 64]) raise a typed error; a prepared list is
  checked against the call's key count and device; array triples passed directly to the op are
  prepared once and kept in a bounded cache."""
  import torch
  from faster_weathernext_amd import hip_attn
  tp = np.array([0, 1, 2], np.int32)
  kb = np.array([0, 1], np.int32)
  with pytest.raises(ValueError, match="128 x 128"):
    hip_attn.TileList(tp, kb, np.zeros((2, 64), np.uint32), 256, device="cpu")
  bits = np.zeros((2, nat.BLOCK, nat.BLOCK // 32), np.uint32)
  bits[:, :, 0] = 1
  tl = hip_attn.TileList(tp, kb, bits, 256, device="cpu")
  with pytest.raises(ValueError, match="columns"):
    hip_attn._as_tiles(tl, 255, torch.device("cpu"))
  with pytest.raises(ValueError, match="lives on"):
    hip_attn._as_tiles(tl, 256, torch.device("cuda", 0))
  assert hip_attn._as_tiles(tl, 256, torch.device("cpu")) is tl
  triples = [(tp.copy(), kb.copy(), bits.copy()) for _ in range(hip_attn.CACHE_LISTS + 2)]
  first = hip_attn._as_tiles(triples[0], 256, torch.device("cpu"))
  assert hip_attn._as_tiles(triples[0], 256, torch.device("cpu")) is first  # prepared once
  for t in triples[1:]:
    hip_attn._as_tiles(t, 256, torch.device("cpu"))
  assert len(hip_attn._cache) == hip_attn.CACHE_LISTS
  assert hip_attn._as_tiles(triples[0], 256, torch.device("cpu")) is not first  # evicted, rebuilt


def test_noalloc_forward_rejects_schedules_beyond_the_static_scratch():
  """fwn_attn_fwd_launch_noalloc checks the split schedule's scratch need against FWN_SCRATCH_BYTES
  before any HIP call, and names the limit in its error."""
  from faster_weathernext_amd import hip_attn
  nb = 130
  tp = np.concatenate([[0], nb + np.arange(nb, dtype=np.int32)]).astype(np.int32)
  kb = np.concatenate([np.arange(nb), np.arange(1, nb)]).astype(np.int32)
  bits = np.full((len(kb), nat.BLOCK, nat.BLOCK // 32), 0xFFFFFFFF, np.uint32)
  n = nb * nat.BLOCK
  tl = hip_attn.TileList(tp, kb, bits, n, device="cpu", max_item_tiles=1)  # block 0: 130 partial slots
  desc = nat.AttnDesc(4, n, 8, 128, nat.BF16, 0.1, n * 1024, 1024, 128, 0, 0, 0)
  size = ctypes.c_uint64(0)
  nat.check(nat.lib().fwn_attn_workspace_size(desc, tl.struct, ctypes.byref(size)))
  assert size.value == 130 * 4 * 8 * 128 * (2 * 128 + 2) * 4 > nat.SCRATCH_BYTES
  rc = nat.lib().fwn_attn_fwd_launch_noalloc(desc, 256, 256, 256, tl.struct, 256, None, None)
  assert rc == nat.ERR_INVALID_ARG
  assert b"static scratch holds 67108864" in nat.lib().fwn_last_error()
  bad = nat.AttnDesc(4, n, 8, 96, nat.BF16, 0.1, n * 1024, 1024, 128, 0, 0, 0)  # head_dim 96 is not built
  assert nat.lib().fwn_attn_fwd_launch_noalloc(bad, 256, 256, 256, tl.struct, 256, None, None) == nat.ERR_UNSUPPORTED


def _ds_map(fwd, tr, unit_keys=16):
  tp, kb, bits = fwd
  tpt, kbt, bitst = tr
  ubase = np.zeros(max(len(kb), 1), np.int32)
  tmap = np.zeros((max(len(kbt), 1), 2), np.int32)
  n_units = np.zeros(1, np.int64)
  status = nat.lib().fwn_tiles_ds_map(len(tp) - 1, nat.ptr(tp), nat.ptr(kb), nat.ptr(bits), nat.ptr(tpt),
                                      nat.ptr(kbt), nat.ptr(bitst), unit_keys, nat.ptr(ubase), nat.ptr(tmap),
                                      nat.ptr(n_units))
  return status, ubase[:len(kb)], tmap[:len(kbt)], int(n_units[0])


@pytest.mark.parametrize("unit_keys", [16, 32])
@pytest.mark.parametrize("symmetric", [True, False])
def test_ds_map_numbers_units_from_the_dense_mask(symmetric, unit_keys):
  # The dS exchange: unit (query group r, key block u of unit_keys keys) of forward tile (qb, kb)
  # exists when the dense mask has a valid element in rows 32r.. x columns unit_keys * u.. of the
  # tile; units are numbered tile by tile in list order, by bit (128 / unit_keys) r + u. The
  # dK/dV kernel's unit for query group c and key block kg of transposed tile (kb, qb) must be
  # that same unit (bit (128 / unit_keys) c + kg).
  n = 700
  m = _random_mask(n, 0.02, 5, symmetric=symmetric)
  fwd = fwn.build_tile_mask(m)
  tr = fwd if symmetric else fwn.build_tile_mask(m.T.tocsr())
  status, ubase, tmap, n_units = _ds_map(fwd, tr, unit_keys)
  assert status == nat.OK
  per = 128 // unit_keys  # units per 32-row group
  dense = np.zeros((6 * 128, 6 * 128), bool)
  dense[:n, :n] = m.toarray()
  tp, kb, _ = fwd
  qb_of = np.repeat(np.arange(len(tp) - 1), np.diff(tp))
  words, want_base, total = {}, [], 0
  for t in range(len(kb)):
    blk = dense[128 * qb_of[t]:128 * qb_of[t] + 128, 128 * kb[t]:128 * kb[t] + 128]
    word = 0
    for r in range(4):
      for u in range(per):
        if blk[32 * r:32 * r + 32, unit_keys * u:unit_keys * (u + 1)].any():
          word |= 1 << (per * r + u)
    words[(qb_of[t], kb[t])] = (total, word)
    want_base.append(total)
    total += bin(word).count("1")
  np.testing.assert_array_equal(ubase, want_base)
  assert n_units == total
  tpt, kbt, _ = tr
  kb_of = np.repeat(np.arange(len(tpt) - 1), np.diff(tpt))
  for t in range(len(kbt)):
    base, word = words[(kbt[t], kb_of[t])]
    assert tmap[t, 0] == base and int(tmap[t, 1].view(np.uint32)) == word
    keys = dense.T[128 * kb_of[t]:128 * kb_of[t] + 128, 128 * kbt[t]:128 * kbt[t] + 128]
    for kg in range(per):
      for c in range(4):
        live = keys[unit_keys * kg:unit_keys * (kg + 1), 32 * c:32 * c + 32].any()
        assert live == bool(word >> (per * c + kg) & 1)


def test_ds_map_rejects_lists_that_are_not_transposes():
  m = _random_mask(500, 0.02, 9)
  fwd = fwn.build_tile_mask(m)
  tr = fwn.build_tile_mask(m.T.tocsr())
  assert _ds_map(fwd, tr)[0] == nat.OK
  assert _ds_map(fwd, tr, 24)[0] == nat.ERR_INVALID_ARG  # 16 or 32 keys per unit
  assert _ds_map(fwd, fwd)[0] == nat.ERR_TILES  # not symmetric
  assert "transpose" in nat.lib().fwn_last_error().decode()
  tp, kb, bits = tr
  flipped = bits.copy()
  flipped[len(kb) // 2, 5, 0] ^= np.uint32(1 << 3)  # one bit
  assert _ds_map(fwd, (tp, kb, flipped))[0] == nat.ERR_TILES
  fewer = np.minimum(tp, len(kb) - 1)  # the last tile dropped
  assert _ds_map(fwd, (fewer, kb[:-1], bits[:-1]))[0] == nat.ERR_TILES


def test_ds_launchers_validate_before_launching():
  L = nat.lib()
  F = FAKE
  tiles = _tiles()
  dmap, dmap32 = nat.DsMap(10, F, F, 16, 0), nat.DsMap(10, F, F, 32, 0)
  bf, f32 = _desc(dtype=nat.BF16, stride_b=300 * 128, stride_n=128, stride_h=64), _desc()
  need, need32 = 1 * 2 * 10 * 1024, 1 * 2 * 10 * 4096
  n = ctypes.c_uint64(0)
  assert L.fwn_attn_ds_bytes(bf, dmap, ctypes.byref(n)) == nat.OK and n.value == need
  assert L.fwn_attn_ds_bytes(f32, dmap32, ctypes.byref(n)) == nat.OK and n.value == need32
  assert L.fwn_attn_ds_bytes(f32, nat.DsMap(10, F, F, 8, 0), ctypes.byref(n)) == nat.ERR_INVALID_ARG
  # a map of the other dtype's unit size
  assert L.fwn_attn_bwd_dq_ds_launch(f32, F, F, need32, tiles, dmap, F, None, 0, None) == nat.ERR_INVALID_ARG
  assert L.fwn_attn_bwd_dkv_ds_launch(bf, F, F, F, F, F, F, tiles, dmap32, F, F, F, need32, None, 0,
                                      None) == nat.ERR_INVALID_ARG
  # a dS buffer too small, misaligned or missing; a (batch, head) slice of units past 2 GiB
  assert L.fwn_attn_bwd_dq_ds_launch(bf, F, F, need - 1, tiles, dmap, F, None, 0, None) == nat.ERR_INVALID_ARG
  assert L.fwn_attn_bwd_dq_ds_launch(f32, F, F, need32 - 1, tiles, dmap32, F, None, 0, None) == nat.ERR_INVALID_ARG
  assert L.fwn_attn_bwd_dq_ds_launch(bf, F, F + 16, need, tiles, dmap, F, None, 0, None) == nat.ERR_INVALID_ARG
  assert L.fwn_attn_bwd_dq_ds_launch(bf, F, None, need, tiles, dmap, F, None, 0, None) == nat.ERR_INVALID_ARG
  assert L.fwn_attn_bwd_dq_ds_launch(bf, F, F, 1 << 40, tiles, nat.DsMap(1 << 21, F, F, 16, 0), F, None, 0,
                                     None) == nat.ERR_INVALID_ARG
  assert L.fwn_attn_bwd_dq_ds_launch(f32, F, F, 1 << 40, tiles, nat.DsMap(1 << 19, F, F, 32, 0), F, None, 0,
                                     None) == nat.ERR_INVALID_ARG
  assert L.fwn_attn_bwd_dq_ds_launch(bf, F, F, need, tiles, nat.DsMap(10, None, F, 16, 0), F, None, 0,
                                     None) == nat.ERR_INVALID_ARG
  assert L.fwn_attn_bwd_dkv_ds_launch(bf, F, F, F, F, F, F, tiles, nat.DsMap(10, F, None, 16, 0), F, F, F, need, None,
                                      0, None) == nat.ERR_INVALID_ARG
  # the bf16 dq kernel needs the forward list's half bits (the float32 one does not)
  t1 = nat.Tiles(3, 1, F, F, F, F, 3, 0, 0, 0, F, None, None)
  assert L.fwn_attn_bwd_dq_ds_launch(bf, F, F, need, t1, dmap, F, None, 0, None) == nat.ERR_TILES


def test_split_precision_is_validated():
  """FWN_PREC_BF16X3 takes float32 tensors; the backward launchers and the scratch forward take
  FWN_PREC_NATIVE only; unknown precisions are refused. All before any HIP call. The workspace
  adds the split k and v (2 * batch * heads * n * head_dim * 4 bytes) after the partial slots."""
  L = nat.lib()
  F = FAKE
  tiles = _tiles()
  x3 = _desc(precision=nat.PREC_BF16X3)
  n = ctypes.c_uint64(0)
  assert L.fwn_attn_workspace_size(x3, tiles, ctypes.byref(n)) == nat.OK
  assert n.value == 3 * (1 * 2 * 300 * 64 * 4)
  split = _tiles(n_items=5, n_parts=3, n_split=1, split=F)
  assert L.fwn_attn_workspace_size(x3, split, ctypes.byref(n)) == nat.OK
  parts = 3 * 1 * 2 * 128 * (2 * 64 + 2) * 4
  assert n.value == ((parts + 255) // 256) * 256 + 3 * (2 * 300 * 64 * 4)
  # a workspace without room for the split tensors is refused
  assert L.fwn_attn_fwd_launch(x3, F, F, F, split, F, None, F, n.value - 1, None) == nat.ERR_INVALID_ARG
  assert L.fwn_attn_fwd_launch(x3, F, F, F, tiles, F, None, F, 3 * (2 * 300 * 64 * 4) - 1,
                               None) == nat.ERR_INVALID_ARG
  assert L.fwn_attn_fwd_launch(x3, F, F, F, tiles, F, None, None, 0, None) == nat.ERR_INVALID_ARG
  for bad, code in ((_desc(dtype=nat.BF16, precision=nat.PREC_BF16X3), nat.ERR_UNSUPPORTED),
                    (_desc(precision=2), nat.ERR_UNSUPPORTED), (_desc(precision=-1), nat.ERR_UNSUPPORTED)):
    assert L.fwn_attn_fwd_launch(bad, F, F, F, tiles, F, None, None, 0, None) == code
    assert L.fwn_attn_workspace_size(bad, tiles, ctypes.byref(n)) == code
  assert L.fwn_attn_bwd_dq_launch(x3, F, F, F, F, F, F, tiles, F, None, 0, None) == nat.ERR_UNSUPPORTED
  assert L.fwn_attn_bwd_dkv_launch(x3, F, F, F, F, F, F, tiles, F, F, None, 0, None) == nat.ERR_UNSUPPORTED
  assert "NATIVE" in L.fwn_last_error().decode()
  # the dS-exchange launchers take bf16x3 with float32-sized (32-key) units and its workspace
  dmap, dmap16 = nat.DsMap(10, F, F, 32, 0), nat.DsMap(10, F, F, 16, 0)
  assert L.fwn_attn_bwd_dkv_ds_launch(x3, F, F, F, F, F, F, tiles, dmap16, F, F, F, 1 << 20, None, 0,
                                      None) == nat.ERR_INVALID_ARG
  assert L.fwn_attn_bwd_dq_ds_launch(x3, F, F, 1 << 20, tiles, dmap, F, None, 0, None) == nat.ERR_INVALID_ARG
  assert "workspace" in L.fwn_last_error().decode()
  assert L.fwn_attn_fwd_launch_noalloc(x3, F, F, F, tiles, F, None, None) == nat.ERR_UNSUPPORTED


def test_split_precision_python_options():
  import torch
  from faster_weathernext_amd import hip_attn, patch
  with pytest.raises(ValueError):
    fwn.enable(force=True, precision="tf32")
  fwn.enable(force=True, precision="bf16x3")
  try:
    assert fwn.TiledMHA(16, 2, 8, None, device="cpu").precision == "bf16x3"
    assert fwn.TiledMHA(16, 2, 8, None, device="cpu", dtype=torch.bfloat16).precision == "native"
    assert fwn.TiledMHA(16, 2, 8, None, device="cpu", precision="native").precision == "native"
  finally:
    fwn.disable()
  assert patch.OPTIONS.precision is None
  assert hip_attn._precision("bf16x3", torch.float32) == nat.PREC_BF16X3
  assert hip_attn._precision("native", torch.bfloat16) == nat.PREC_NATIVE
  with pytest.raises(TypeError):
    hip_attn._precision("bf16x3", torch.bfloat16)
  with pytest.raises(ValueError):
    hip_attn._precision("tf32", torch.float32)


def test_reference_keyword_arguments():
  """tiled_flash_attention takes the reference's keywords (pallas_attn.py:317-320): Triton tuning
  values are accepted, other tile sizes and the CPU interpreter are refused with ValueError
  before any GPU work."""
  from faster_weathernext_amd import hip_attn
  hip_attn._reference_options(128, 128, False)
  hip_attn._reference_options(None, None, False)
  for args in ((64, None, False), (None, 32, False), (None, None, True)):
    with pytest.raises(ValueError):
      hip_attn._reference_options(*args)
  import inspect
  params = inspect.signature(fwn.tiled_flash_attention).parameters
  for name in ("scale", "strict_fp32", "tiles_t", "block_q", "block_k", "num_warps", "num_stages", "bwd_num_warps",
               "bwd_split", "interpret"):
    assert name in params, name


# The reference's Options fields and defaults (patch.py:50-79).
REFERENCE_OPTIONS = dict(attention="auto", replace_attention=True, reorder=True, strict_fp32=False, attn_chunk=512,
                         grid_chunk=32768, edge_chunk=65536, layer_loop=True, remat=False, sequential_samples=False)


def test_enable_accepts_every_reference_option():
  from faster_weathernext_amd import patch
  try:
    opts = fwn.enable(force=True, **REFERENCE_OPTIONS)
    for key, value in REFERENCE_OPTIONS.items():
      assert getattr(opts, key) == value, key
    opts = fwn.enable(force=True, strict_fp32=True, attn_chunk=256, remat=True)
    assert opts.strict_fp32 is True and opts.attn_chunk == 256
  finally:
    fwn.disable()
  assert patch.OPTIONS.strict_fp32 is False


def test_strict_fp32_selects_the_ieee_kernels():
  """The reference's dot choice (pallas_attn.py:336-341) with torch's float32 matmul precision in
  place of JAX's: "highest" -> IEEE products; "high" / "medium" -> bf16x3 unless strict_fp32."""
  import torch
  from faster_weathernext_amd import patch
  resolve = patch.resolve_precision
  saved = torch.get_float32_matmul_precision()
  try:
    torch.set_float32_matmul_precision("highest")
    assert resolve(None, torch.float32, False) == "native"
    assert resolve(None, torch.float32, True) == "native"
    for knob in ("high", "medium"):
      torch.set_float32_matmul_precision(knob)
      assert resolve(None, torch.float32, False) == "bf16x3"
      assert resolve(None, torch.float32, True) == "native"
      assert resolve("native", torch.float32, False) == "native"
      assert resolve(None, torch.bfloat16, False) == "native"
      with pytest.raises(ValueError):
        resolve("bf16x3", torch.float32, True)
      # The enable() option reaches the modules built afterwards.
      try:
        fwn.enable(force=True, strict_fp32=True)
        assert fwn.TiledMHA(16, 2, 8, None, device="cpu").precision == "native"
        assert resolve(None, torch.float32) == "native"
      finally:
        fwn.disable()
      assert fwn.TiledMHA(16, 2, 8, None, device="cpu").precision == "bf16x3"
  finally:
    torch.set_float32_matmul_precision(saved)
  with pytest.raises(TypeError):
    resolve("bf16x3", torch.bfloat16)
  with pytest.raises(ValueError):
    resolve("tf32", torch.float32)


def test_build_tile_mask_takes_the_reference_signature():
  """build_tile_mask(mask, block_q, block_k) as the reference's (pallas_attn.py:85): 128 x 128 is
  what the kernels use; the reference's 64 x 32 default is refused rather than misread."""
  from scipy import sparse
  m = sparse.identity(300, dtype=bool, format="csr")
  a = fwn.build_tile_mask(m)
  b = fwn.build_tile_mask(m, 128, 128)
  for x, y in zip(a, b):
    np.testing.assert_array_equal(x, y)
  with pytest.raises(ValueError):
    fwn.build_tile_mask(m, 64, 32)


def test_output_strides_must_not_overlap():
  """Outputs written through strides whose (batch, row, head) rows overlap would race: the
  forward checks the o strides, the dq/dk/dv launchers the q strides, before any HIP call.
  Inputs may overlap (read only): a forward whose q, k, v broadcast over the batch (stride 0)
  with a proper o passes validation."""
  L = nat.lib()
  F = FAKE
  tiles = _tiles()
  # head-major with stride_n == stride_h == head_dim: head 1 row 0 is head 0 row 1
  bad = _desc(stride_b=300 * 128, stride_n=64, stride_h=64)
  assert L.fwn_attn_fwd_launch(bad, F, F, F, tiles, F, None, None, 0, None) == nat.ERR_INVALID_ARG
  assert "overlap" in L.fwn_last_error().decode()
  assert L.fwn_attn_bwd_dq_launch(bad, F, F, F, F, F, F, tiles, F, None, 0, None) == nat.ERR_INVALID_ARG
  assert L.fwn_attn_bwd_dkv_launch(bad, F, F, F, F, F, F, tiles, F, F, None, 0, None) == nat.ERR_INVALID_ARG
  # batches overlapping (stride_b smaller than a batch's extent)
  bad_b = _desc(batch=2, stride_b=128, stride_n=128, stride_h=64)
  assert L.fwn_attn_bwd_dq_launch(bad_b, F, F, F, F, F, F, tiles, F, None, 0, None) == nat.ERR_INVALID_ARG
  # broadcast inputs (stride_b 0), disjoint o strides: passes validation (fails later at the tiles)
  bcast = _desc(batch=2, stride_b=0, stride_n=128, stride_h=64, ostride_b=300 * 128, ostride_n=128, ostride_h=64)
  assert L.fwn_attn_fwd_launch(bcast, F, F, F, _tiles(n_blocks=5), F, None, None, 0, None) == nat.ERR_TILES
  # the packed qkv views are disjoint
  packed = _desc(stride_b=300 * 3 * 2 * 64, stride_n=3 * 2 * 64, stride_h=64)
  assert L.fwn_attn_fwd_launch(packed, F, F, F, _tiles(n_blocks=5), F, None, None, 0, None) == nat.ERR_TILES


def test_mesh_transformer_refuses_caller_tiles_without_transpose():
  """A non-symmetric adjacency with caller-built tiles and no tiles_t would make the backward walk
  the forward list as its own transpose; the constructor refuses it before building any layer."""
  n = 200
  adj = sparse.random(n, n, density=0.02, random_state=3, format="csr").astype(bool)
  assert (adj != adj.T).nnz
  mask = fwn.khop_mask(adj, 2)
  tiles = fwn.TileList.from_mask(mask, device="cpu")
  with pytest.raises(ValueError, match="tiles_t"):
    fwn.MeshTransformer(num_layers=1, d_model=16, num_heads=2, key_size=8, ffw_hidden=32, cond_size=4,
                        reorder=False, device="cpu", tiles=tiles, adjacency=adj, k_hop=2)


def test_ds_maps_live_as_long_as_their_transposed_list():
  import gc
  m = _random_mask(300, 0.05, 5, symmetric=True)
  tl = fwn.TileList.from_mask(m, device="cpu")
  assert tl.ds_map(tl) is not None and tl.ds_map(tl) is tl.ds_map(tl)
  other = fwn.TileList.from_mask(m, device="cpu")
  assert other.ds_map(tl) is not None
  maps = other._ds_maps[16]
  assert len(maps) == 1
  del tl
  gc.collect()
  assert len(maps) == 0


def test_delta_launch_refuses_a_grid_past_32_bits():
  """The delta kernel's one-dimensional grid holds (n / 8) x batch workgroups at most: a call past
  2^31 of them is refused before any HIP call."""
  L = nat.lib()
  n, batch = 1 << 15, 1 << 20
  big = _desc(batch=batch, n=n, heads=1, head_dim=128, stride_b=n * 128, stride_n=128, stride_h=128)
  assert L.fwn_attn_bwd_delta_launch(big, FAKE, FAKE, FAKE, None) == nat.ERR_INVALID_ARG
  assert "too large" in L.fwn_last_error().decode()
