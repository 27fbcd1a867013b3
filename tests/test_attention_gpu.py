"""GPU parity tests: the HIP kernels (through the C ABI) against the CPU oracle.

Bars: rel RMS <= 1e-5 at float32 and <= 5e-3 at bfloat16 per output tensor, plus
the reference's own unit-test metric max|got - ref| / max|ref| (tests/test_pallas_kernel.py:54,
98: 1e-5 at full precision). bfloat16 cases compare against the float64 oracle evaluated on the
bf16-rounded inputs. Small cases use the dense oracle; model-scale cases (refinement-6 mesh) use the
exact sampled oracle on a seeded subset of rows and keys plus size-independent identities.
"""

import numpy as np
import pytest
import torch
from scipy import sparse

import faster_weathernext_amd as fwn
from faster_weathernext_amd import _native as nat
from oracle import attention as A

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = {torch.float32: 1e-5, torch.bfloat16: 5e-3}
MAXTOL = {torch.float32: 1e-5, torch.bfloat16: 3e-2}


def _random_mask(n, density, seed, symmetric=False, identity=True):
  m = sparse.random(n, n, density=density, random_state=seed, format="csr").astype(bool)
  if symmetric:
    m = m + m.T
  if identity:
    m = m + sparse.identity(n, dtype=bool, format="csr")
  return m.tocsr().astype(bool)


def _rounded(x, dtype):
  """Inputs as the kernel sees them (bf16 rounding, round to nearest even), back in float32."""
  return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(dtype).float().numpy()


def _dev(x, dtype, grad=False):
  t = torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(DEV).to(dtype)
  return t.requires_grad_(grad)


def _np(t):
  return t.detach().float().cpu().numpy()


def _run(q, k, v, do, tiles, scale, dtype, tiles_t=None):
  qt, kt, vt = (_dev(x, dtype, do is not None) for x in (q, k, v))
  out = fwn.tiled_flash_attention(qt, kt, vt, tiles, scale=scale, tiles_t=tiles_t)
  res = {"out": _np(out)}
  if do is not None:
    out.backward(_dev(do, dtype))
    res.update(dq=_np(qt.grad), dk=_np(kt.grad), dv=_np(vt.grad))
  torch.cuda.synchronize()
  return res


def _check(got, ref, dtype, what):
  rr, mr = A.rel_rms(got, ref), A.max_rel_err(got, ref)
  assert rr <= TOL[dtype], (what, rr, mr)
  assert mr <= MAXTOL[dtype], (what, rr, mr)


# ---------------------------------------------------------------------------------------------
# configuration 1 (golden vectors)


def test_c1_golden_fp32():
  g = np.load(__file__.replace("test_attention_gpu.py", "golden/c1_r3_2hop.npz"))
  n = g["q"].shape[1]
  mask = sparse.csr_matrix((np.ones(len(g["indices"]), bool), g["indices"], g["indptr"]), shape=(n, n))
  tiles = fwn.TileList.from_mask(mask)
  scale = float(g["scale"])
  res = _run(g["q"], g["k"], g["v"], g["do"], tiles, scale, torch.float32)
  for name in ("out", "dq", "dk", "dv"):
    _check(res[name], g[name], torch.float32, name)
  out, lse = fwn.attention_forward(_dev(g["q"], torch.float32), _dev(g["k"], torch.float32),
                                   _dev(g["v"], torch.float32), tiles, scale)
  np.testing.assert_allclose(_np(lse), g["lse"], rtol=0, atol=2e-5)


def test_c1_matches_reference_chunked_path():
  """Against the restated reference XLA chunked path (patch.py:106-162) at float32."""
  g = np.load(__file__.replace("test_attention_gpu.py", "golden/c1_r3_2hop.npz"))
  n = g["q"].shape[1]
  mask = sparse.csr_matrix((np.ones(len(g["indices"]), bool), g["indices"], g["indptr"]), shape=(n, n))
  scale = float(g["scale"])
  starts, bits, window, n_kv = A.build_chunked_mask(mask, 512)
  ref = A.chunked_attention(g["q"], g["k"], g["v"], starts, bits, window, n_kv, 512, scale)
  refg = A.chunked_attention_grads(g["q"], g["k"], g["v"], g["do"], starts, bits, window, n_kv, 512, scale)
  res = _run(g["q"], g["k"], g["v"], g["do"], fwn.TileList.from_mask(mask), scale, torch.float32)
  assert A.rel_rms(res["out"], ref) <= 1e-5
  for name, r in zip(("dq", "dk", "dv"), refg):
    assert A.rel_rms(res[name], r) <= 1e-5, name


def test_c1_bf16():
  g = np.load(__file__.replace("test_attention_gpu.py", "golden/c1_r3_2hop.npz"))
  n = g["q"].shape[1]
  mask = sparse.csr_matrix((np.ones(len(g["indices"]), bool), g["indices"], g["indptr"]), shape=(n, n))
  q, k, v, do = (_rounded(g[x], torch.bfloat16) for x in ("q", "k", "v", "do"))
  scale = float(g["scale"])
  res = _run(q, k, v, do, fwn.TileList.from_mask(mask), scale, torch.bfloat16)
  dense = mask.toarray()
  _check(res["out"], A.dense_attention(q, k, v, dense, scale), torch.bfloat16, "out")
  for name, r in zip(("dq", "dk", "dv"), A.dense_grads(q, k, v, do, dense, scale)):
    _check(res[name], r, torch.bfloat16, name)


# ---------------------------------------------------------------------------------------------
# the reference's kernel tests (tests/test_pallas_kernel.py), same generators and seeds


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("batch", [1, 2])
def test_matches_dense_reference(batch, dtype):
  rng = np.random.default_rng(0)
  n, h, d = 300, 2, 64
  q, k, v = (_rounded(rng.standard_normal((batch, n, h, d)), dtype) for _ in range(3))
  m = _random_mask(n, 0.1, 1)
  res = _run(q, k, v, None, fwn.TileList.from_mask(m), d ** -0.5, dtype)
  ref = A.dense_attention(q, k, v, m.toarray(), d ** -0.5)
  for b in range(batch):
    _check(res["out"][b], ref[b], dtype, ("out", b))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("symmetric", [True, False])
@pytest.mark.parametrize("batch", [1, 2])
@pytest.mark.parametrize("d", [64, 128])
def test_grads_match_dense_reference(d, batch, symmetric, dtype):
  rng = np.random.default_rng(2)
  n, h = 300, 2
  q, k, v, do = (_rounded(rng.standard_normal((batch, n, h, d)), dtype) for _ in range(4))
  m = _random_mask(n, 0.08, 3, symmetric=symmetric)
  tiles = fwn.TileList.from_mask(m)
  tiles_t = None if symmetric else fwn.TileList.from_mask(m.T.tocsr())
  res = _run(q, k, v, do, tiles, d ** -0.5, dtype, tiles_t)
  refs = A.dense_grads(q, k, v, do, m.toarray(), d ** -0.5)
  for b in range(batch):
    for name, r in zip(("dq", "dk", "dv"), refs):
      _check(res[name][b], r[b], dtype, (name, b))


def test_nonsymmetric_mask_needs_transposed_tiles():
  rng = np.random.default_rng(4)
  n, h, d = 130, 1, 32
  q, k, v, do = (rng.standard_normal((1, n, h, d)).astype(np.float32) for _ in range(4))
  m = _random_mask(n, 0.1, 5)
  tiles = fwn.TileList.from_mask(m)
  ref = A.dense_grads(q, k, v, do, m.toarray(), d ** -0.5)[1]
  wrong = _run(q, k, v, do, tiles, d ** -0.5, torch.float32)["dk"]
  assert A.max_rel_err(wrong, ref) > 1e-2
  right = _run(q, k, v, do, tiles, d ** -0.5, torch.float32, fwn.TileList.from_mask(m.T.tocsr()))["dk"]
  assert A.max_rel_err(right, ref) < 1e-5


# ---------------------------------------------------------------------------------------------
# shapes and edge cases


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("d", [32, 64, 128])
@pytest.mark.parametrize("n", [100, 257, 512])
def test_head_dims_and_ragged_sizes(n, d, dtype):
  rng = np.random.default_rng(n + d)
  h = 3
  q, k, v, do = (_rounded(rng.standard_normal((1, n, h, d)), dtype) for _ in range(4))
  m = _random_mask(n, 0.05, 6, symmetric=True)
  res = _run(q, k, v, do, fwn.TileList.from_mask(m), d ** -0.5, dtype)
  dense = m.toarray()
  _check(res["out"], A.dense_attention(q, k, v, dense, d ** -0.5), dtype, "out")
  for name, r in zip(("dq", "dk", "dv"), A.dense_grads(q, k, v, do, dense, d ** -0.5)):
    _check(res[name], r, dtype, name)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_fully_valid_tiles(dtype):
  """A dense mask: every tile takes the no-mask path."""
  rng = np.random.default_rng(7)
  n, h, d = 256, 2, 64
  q, k, v, do = (_rounded(rng.standard_normal((1, n, h, d)), dtype) for _ in range(4))
  m = sparse.csr_matrix(np.ones((n, n), bool))
  tiles = fwn.TileList.from_mask(m)
  assert tiles.n_tiles == 4
  res = _run(q, k, v, do, tiles, d ** -0.5, dtype)
  dense = m.toarray()
  _check(res["out"], A.dense_attention(q, k, v, dense, d ** -0.5), dtype, "out")
  for name, r in zip(("dq", "dk", "dv"), A.dense_grads(q, k, v, do, dense, d ** -0.5)):
    _check(res[name], r, dtype, name)


def test_rows_without_keys_are_zero_and_finite():
  """Rows with no valid key produce 0 (the reference leaves such rows undefined; none occur in a
  k-hop mask, where every row attends to itself). Other rows are unaffected."""
  rng = np.random.default_rng(8)
  n, h, d = 200, 2, 32
  q, k, v, do = (rng.standard_normal((1, n, h, d)).astype(np.float32) for _ in range(4))
  m = _random_mask(n, 0.05, 9, symmetric=True).tolil()
  empty = [3, 64, 130, 199]
  for r in empty:
    m[r, :] = False
    m[:, r] = False
  m = m.tocsr()
  m.eliminate_zeros()
  res = _run(q, k, v, do, fwn.TileList.from_mask(m), d ** -0.5, torch.float32)
  for name in res:
    assert np.isfinite(res[name]).all(), name
  np.testing.assert_array_equal(res["out"][:, empty], 0.0)
  keep = np.setdiff1d(np.arange(n), empty)
  dense = m.toarray()
  sub = dense[np.ix_(keep, keep)]
  ref = A.dense_attention(q[:, keep], k[:, keep], v[:, keep], sub, d ** -0.5)
  _check(res["out"][:, keep], ref, torch.float32, "out")
  refs = A.dense_grads(q[:, keep], k[:, keep], v[:, keep], do[:, keep], sub, d ** -0.5)
  for name, r in zip(("dq", "dk", "dv"), refs):
    _check(res[name][:, keep], r, torch.float32, name)
    np.testing.assert_array_equal(res[name][:, empty], 0.0)


@pytest.mark.parametrize("case", ["bf16", "f32", "bf16x3"])
@pytest.mark.parametrize("n", [1, 2, 33, 129])
def test_tiny_sequences(n, case):
  """Sequences shorter than one 32-row group, one block plus one row: a single partial tile (or
  two blocks), most of its rows and columns past n. Forward and backward against the dense
  float64 oracle. With so few keys per row dq = scale sum_j dS_ij k_j is a difference of a few
  rounded terms (sum_j dS_ij = 0) and dS = P (dP - delta) a difference of a few products (with
  n = 1, P = 1 and dS = 0 exactly), so dq and dk are held to the rounding bounds of their sums
  (_grad_rounding_bounds, u = 2^-7 in bf16, 2^-14 in float32 and bf16x3); out and dv to the
  usual bars."""
  print(f"tiny n={n} {case}", flush=True)
  dtype = torch.bfloat16 if case == "bf16" else torch.float32
  precision = "bf16x3" if case == "bf16x3" else "native"
  rng = np.random.default_rng(n)
  b, h, d = 2, 2, 64
  q, k, v, do = (_rounded(rng.standard_normal((b, n, h, d)), dtype) for _ in range(4))
  m = _random_mask(n, 0.3, n, symmetric=True)
  tiles = fwn.TileList.from_mask(m)
  qt, kt, vt = (_dev(x, dtype, True) for x in (q, k, v))
  out = fwn.tiled_flash_attention(qt, kt, vt, tiles, scale=d ** -0.5, precision=precision)
  out.backward(_dev(do, dtype))
  torch.cuda.synchronize()
  dense = m.toarray()
  # bf16x3 keeps its own float32 bars (max 2e-5 of max|ref|, tests/test_x3_gpu.py).
  rms, mx = (TOL[dtype], MAXTOL[dtype]) if precision == "native" else (1e-5, 2e-5)

  def check(got, ref, what):
    rr, mr = A.rel_rms(got, ref), A.max_rel_err(got, ref)
    assert rr <= rms and mr <= mx, (what, rr, mr)

  check(_np(out), A.dense_attention(q, k, v, dense, d ** -0.5), "out")
  ref_dq, ref_dk, ref_dv = A.dense_grads(q, k, v, do, dense, d ** -0.5)
  bq, bk = _grad_rounding_bounds(q, k, v, do, _np(out), dense, d ** -0.5)
  u = 2.0 ** -7 if dtype == torch.bfloat16 else 2.0 ** -14
  for t, r, b, name in ((qt, ref_dq, bq, "dq"), (kt, ref_dk, bk, "dk")):
    ratio = np.abs(_np(t.grad) - r) / (u * b + 1e-30)
    assert ratio.max() <= 1.0, (name, ratio.max())
  check(_np(vt.grad), ref_dv, "dv")


@pytest.mark.parametrize("exchange", [True, False])
@pytest.mark.parametrize("case", ["bf16", "f32", "bf16x3"])
def test_mask_without_valid_elements(case, exchange, monkeypatch):
  """A mask with no valid element at all has no tiles (every array of the list empty): every
  row is a row without keys, so the output and every gradient are zero, with the dS exchange
  and with the recomputing backward."""
  print(f"empty mask {case} exchange={exchange}", flush=True)
  monkeypatch.setattr(fwn.hip_attn, "DS_EXCHANGE", exchange)
  dtype = torch.bfloat16 if case == "bf16" else torch.float32
  precision = "bf16x3" if case == "bf16x3" else "native"
  rng = np.random.default_rng(3)
  n, h, d = 300, 2, 64
  q, k, v, do = (rng.standard_normal((1, n, h, d)) for _ in range(4))
  tiles = fwn.TileList.from_mask(sparse.csr_matrix((n, n), dtype=bool))
  assert tiles.n_tiles == 0
  qt, kt, vt = (_dev(x, dtype, True) for x in (q, k, v))
  out = fwn.tiled_flash_attention(qt, kt, vt, tiles, scale=d ** -0.5, precision=precision)
  out.backward(_dev(do, dtype))
  torch.cuda.synchronize()
  for t in (out, qt.grad, kt.grad, vt.grad):
    np.testing.assert_array_equal(_np(t), 0.0)


def _group_pattern_mask(seed):
  """n = 512 mask built from 32 x 32 groups so that the group skipping meets every case: per
  tile, waves (row groups) with different live column groups, waves with none, column groups
  live for no wave (not copied), full groups, groups holding a single element, and
  non-symmetric structure (the dK/dV list is the transposed mask's). Every row has a key."""
  rng = np.random.default_rng(seed)
  m = np.zeros((512, 512), bool)

  def group(rb, cb, rg, cg, density=None, single=None):
    r0, c0 = 128 * rb + 32 * rg, 128 * cb + 32 * cg
    if single is not None:
      m[r0 + single[0], c0 + single[1]] = True
      return
    g = rng.random((32, 32)) < density if density < 1 else np.ones((32, 32), bool)
    g[np.arange(32), rng.integers(0, 32, 32)] = True  # every row of the group has a key
    m[r0:r0 + 32, c0:c0 + 32] |= g

  for rg in range(4):                       # tile (0, 0): one different column group per wave
    group(0, 0, rg, (rg + 1) % 4, density=0.3)
  group(0, 1, 2, 0, single=(5, 3))          # tile (0, 1): only wave 2, two single elements
  group(0, 1, 2, 3, single=(20, 31))
  group(1, 1, 1, 2, density=1.0)            # tile (1, 1): one full group ...
  for rg in (0, 2, 3):                      # ... and single elements for the other waves
    for r in range(32):
      m[128 + 32 * rg + r, 128 + (r * 7) % 32] = True
  for rg in range(4):                       # tile (2, 3): column group 1 dead for every wave
    for cg in (0, 2, 3):
      group(2, 3, rg, cg, density=0.2)
  for r in range(32):                       # tile (3, 0): wave 0 only, one key per row
    m[384 + r, 96 + r] = True
  for rg in (1, 2, 3):                      # tile (3, 2): waves 1-3, column group 1
    group(3, 2, rg, 1, density=0.25)
  assert m.any(1).all()
  return sparse.csr_matrix(m)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("d", [64, 128])
def test_group_skipping_patterns(d, dtype):
  print(f"group patterns d={d} {dtype}", flush=True)
  m = _group_pattern_mask(21)
  tiles, tiles_t = fwn.TileList.from_mask(m), fwn.TileList.from_mask(m.T.tocsr())
  # the designed tiles skip what they should: (0, 1) has only wave 2's bits, (2, 3) no column 1
  kb = tiles.col.cpu().numpy()
  ptr = tiles.ptr.cpu().numpy()
  g01 = tiles.groups_host[ptr[0] + int(np.flatnonzero(kb[ptr[0]:ptr[1]] == 1)[0])]
  assert g01 == (1 << 8) | (1 << 11)
  g23 = tiles.groups_host[ptr[2] + int(np.flatnonzero(kb[ptr[2]:ptr[3]] == 3)[0])]
  assert g23 & 0x2222 == 0 and g23 & 0xDDDD == 0xDDDD
  rng = np.random.default_rng(22)
  n, h = 512, 2
  q, k, v, do = (_rounded(rng.standard_normal((1, n, h, d)), dtype) for _ in range(4))
  res = _run(q, k, v, do, tiles, d ** -0.5, dtype, tiles_t)
  dense = m.toarray()
  _check(res["out"], A.dense_attention(q, k, v, dense, d ** -0.5), dtype, "out")
  for name, r in zip(("dq", "dk", "dv"), A.dense_grads(q, k, v, do, dense, d ** -0.5)):
    _check(res[name], r, dtype, name)


def _without_halves(tiles):
  """The same prepared list with its half bits dropped (every half of a live group processed)."""
  import copy
  t = copy.copy(tiles)
  t.struct = nat.Tiles.from_buffer_copy(tiles.struct)
  t.struct.halves = None
  return t


@pytest.mark.parametrize("d", [32, 64, 128])
def test_half_skipping_is_exact(d, monkeypatch):
  """Skipping the 16-column halves of live 32 x 32 groups that hold no valid element (the bf16
  recomputing dQ kernel) only drops terms that are exact zeros: outputs and gradients are bitwise
  those of the same list without half bits, and both match the dense oracle. The designed pattern
  has live groups with one dead half; the random sparse mask has many."""
  print(f"half skipping d={d}", flush=True)
  monkeypatch.setattr(fwn.hip_attn, "DS_EXCHANGE", False)
  dtype = torch.bfloat16
  rng = np.random.default_rng(70 + d)
  for m in (_group_pattern_mask(21), _random_mask(640, 0.004, 71, symmetric=True)):
    n = m.shape[0]
    tiles, tiles_t = fwn.TileList.from_mask(m), fwn.TileList.from_mask(m.T.tocsr())
    hv, g = tiles.halves_host, tiles.groups_host
    live_halves = sum(bin(int(x)).count("1") for x in hv)
    live_groups = sum(bin(int(x) & 0xFFFF).count("1") for x in g)
    assert live_halves < 2 * live_groups  # some live group has a dead half
    q, k, v, do = (_rounded(rng.standard_normal((2, n, 2, d)), dtype) for _ in range(4))
    got = _run(q, k, v, do, tiles, d ** -0.5, dtype, tiles_t)
    ref = _run(q, k, v, do, _without_halves(tiles), d ** -0.5, dtype, _without_halves(tiles_t))
    for name in got:
      np.testing.assert_array_equal(got[name], ref[name], err_msg=name)
    dense = m.toarray()
    _check(got["out"], A.dense_attention(q, k, v, dense, d ** -0.5), dtype, "out")
    for name, r in zip(("dq", "dk", "dv"), A.dense_grads(q, k, v, do, dense, d ** -0.5)):
      _check(got[name], r, dtype, name)


def _run_modes(q, k, v, do, tiles, scale, dtype, tiles_t, monkeypatch):
  """The backward with the dS exchange (the default for bf16) and with the recomputing dQ kernel."""
  got = _run(q, k, v, do, tiles, scale, dtype, tiles_t)
  monkeypatch.setattr(fwn.hip_attn, "DS_EXCHANGE", False)
  ref = _run(q, k, v, do, tiles, scale, dtype, tiles_t)
  monkeypatch.setattr(fwn.hip_attn, "DS_EXCHANGE", True)
  return got, ref


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("d", [32, 64, 128])
@pytest.mark.parametrize("case", ["symmetric", "transposed", "split", "groups"])
def test_ds_exchange_matches_recompute_and_oracle(case, d, dtype, monkeypatch):
  """Backward with the dS exchange: the dK/dV kernel writes every unit of dS (32 x 16 in bf16,
  32 x 32 in float32) and the dQ kernel reads it (5 contractions per tile instead of 7). dK and
  dV come from the same kernel arithmetic as without the exchange, bit for bit; dQ differs from
  the recomputing kernel's only in rounding (S contracted in other MFMA shapes and k orders, and
  in float32 delta subtracted at another point) and both meet the bars against the dense float64
  oracle. Cases: a symmetric mask (one list) with rows and columns without a valid element, a
  non-symmetric mask with its transposed list, split schedules (items of 1 and 3 tiles, so
  partial dQ and dK/dV slots are combined) and the designed group/half patterns
  (non-symmetric)."""
  print(f"ds exchange {case} d={d} {dtype}", flush=True)
  rng = np.random.default_rng(80 + d)
  n, b, h = 700, 2, 2
  tiles_t = None
  if case == "groups":
    m = _group_pattern_mask(22)
    n = m.shape[0]
  else:
    m = _random_mask(n, 0.02, 81, symmetric=case != "transposed")
  if case == "symmetric":
    m = m.tolil()
    for r in (5, 300):
      m[r, :] = False
      m[:, r] = False
    m = m.tocsr()
    m.eliminate_zeros()
  cap = 1 if case == "split" else None
  tiles = fwn.TileList.from_mask(m, max_item_tiles=cap)
  if case in ("transposed", "groups"):
    tiles_t = fwn.TileList.from_mask(m.T.tocsr())
  if case == "split":
    tiles_t = fwn.TileList.from_mask(m, max_item_tiles=3)
    assert tiles.n_split > 0 and tiles_t.n_split > 0
  assert tiles.ds_map(tiles if tiles_t is None else tiles_t, fwn.hip_attn.unit_keys_for(dtype)) is not None
  q, k, v, do = (_rounded(rng.standard_normal((b, n, h, d)), dtype) for _ in range(4))
  got, ref = _run_modes(q, k, v, do, tiles, d ** -0.5, dtype, tiles_t, monkeypatch)
  for name in ("out", "dk", "dv"):
    np.testing.assert_array_equal(got[name], ref[name], err_msg=name)
  # float32: two summation orders of S and dP, then dS = P (dP - delta) with its cancellation,
  # differ by a few units of rounding (about 1e-6 relative rms).
  close = 1e-3 if dtype == torch.bfloat16 else 3e-6
  assert A.rel_rms(got["dq"], ref["dq"]) < close, A.rel_rms(got["dq"], ref["dq"])
  # Rows and columns cleared in the symmetric case get zero gradients; the oracle runs on the rest.
  keep = np.flatnonzero(m.getnnz(1) > 0)
  empty = np.setdiff1d(np.arange(n), keep)
  for name in ("dq", "dk", "dv"):
    np.testing.assert_array_equal(got[name][:, empty], 0.0)
  sub = m.toarray()[np.ix_(keep, keep)]
  xs = (x[:, keep] for x in (q, k, v, do))
  for name, r in zip(("dq", "dk", "dv"), A.dense_grads(*xs, sub, d ** -0.5)):
    for res in (got, ref):
      _check(res[name][:, keep], r, dtype, name)


def _pair_skew_mask(n, heavy, seed):
  """A non-symmetric banded mask whose valid keys crowd into one half of every 128-key block:
  keys 64 * heavy .. 64 * heavy + 63 of a block are valid for every query within 150 rows, the
  other half only on the diagonal and at a few scattered keys (heavy = 2: both halves dense). The bf16 dK/dV kernel gives keys
  16 kg .. 16 kg + 15 of a block to wave kg and pairs waves s and s + 4 on one SIMD, so with
  heavy = 0 the waves 0-3 hold most units of every tile (waves 4-7 then issue the pairs' copies),
  with heavy = 1 the reverse, and with heavy = 2 the pairs mostly tie."""
  rng = np.random.default_rng(seed)
  rows, cols = [], []
  for q in range(n):
    ks = np.arange(max(0, q - 150), min(n, q + 150))
    half = (ks % 128) // 64
    dense = ks[(half == heavy) | (heavy == 2)]
    sparse_ks = ks[(half != heavy) & (heavy != 2)]
    sparse_ks = sparse_ks[rng.random(len(sparse_ks)) < 0.0005]
    sel = np.unique(np.concatenate([dense, sparse_ks, [q]]))
    rows.extend([q] * len(sel))
    cols.extend(sel.tolist())
  return sparse.csr_matrix((np.ones(len(rows), bool), (rows, cols)), shape=(n, n))


@pytest.mark.parametrize("heavy", [0, 1, 2])
def test_ds_exchange_paired_copies(heavy, monkeypatch):
  """The bf16 dK/dV kernel with the dS exchange lets the wave of each SIMD pair with fewer units
  in a tile issue the pair's whole Q/dO copy (and pair 0's copier the lse/delta copy and its
  rescale). On masks that make one half of every pair heavy (both ways) or the pairs tie, dK and
  dV equal the recomputing kernel's, which keeps the fixed split, bit for bit, and every output
  meets the bf16 bars against the dense float64 oracle."""
  print(f"paired copies heavy={heavy}", flush=True)
  n, b, h, d = 700, 1, 2, 128
  m = _pair_skew_mask(n, heavy, 70 + heavy)
  tiles = fwn.TileList.from_mask(m)
  tiles_t = fwn.TileList.from_mask(m.T.tocsr())
  # The forward tile's half bits (bit 8c + kg: query group c, 16-key group kg) count each wave's
  # units in a tile; check that the mask gives the pairs the intended balance: per tile and pair,
  # which of waves s and s + 4 holds more units.
  more = {"lo": 0, "hi": 0, "tie": 0}
  for x in np.asarray(tiles.halves_host).astype(np.uint64).tolist():
    for s in range(4):
      a, c = (bin(x >> g & 0x01010101).count("1") for g in (s, s + 4))
      more["lo" if a > c else "hi" if a < c else "tie"] += 1
  print(more, flush=True)
  if heavy < 2:
    big, small = ("lo", "hi") if heavy == 0 else ("hi", "lo")
    assert more[big] > 2 * (more[small] + more["tie"]), more
  else:
    assert min(more.values()) >= 8, more
  dtype = torch.bfloat16
  rng = np.random.default_rng(90 + heavy)
  q, k, v, do = (_rounded(rng.standard_normal((b, n, h, d)), dtype) for _ in range(4))
  got, ref = _run_modes(q, k, v, do, tiles, d ** -0.5, dtype, tiles_t, monkeypatch)
  for name in ("out", "dk", "dv"):
    np.testing.assert_array_equal(got[name], ref[name], err_msg=name)
  assert A.rel_rms(got["dq"], ref["dq"]) < 1e-3, A.rel_rms(got["dq"], ref["dq"])
  dense = m.toarray()
  _check(got["out"], A.dense_attention(q, k, v, dense, d ** -0.5), dtype, "out")
  for name, r in zip(("dq", "dk", "dv"), A.dense_grads(q, k, v, do, dense, d ** -0.5)):
    _check(got[name], r, dtype, name)


def test_ds_exchange_falls_back_for_a_list_that_is_not_the_transpose(monkeypatch):
  """A non-symmetric mask run without its transposed list (the reference's tiles_t=None) is not
  a transpose pair, so the dS exchange does not apply and the bf16 backward recomputes dQ: dQ
  is right, dK is what the forward list gives (wrong for this mask, as in the reference)."""
  rng = np.random.default_rng(90)
  n, h, d = 300, 1, 64
  dtype = torch.bfloat16
  q, k, v, do = (_rounded(rng.standard_normal((1, n, h, d)), dtype) for _ in range(4))
  m = _random_mask(n, 0.05, 91)
  tiles = fwn.TileList.from_mask(m)
  assert tiles.ds_map(tiles) is None
  got, ref = _run_modes(q, k, v, do, tiles, d ** -0.5, dtype, None, monkeypatch)
  for name in got:
    np.testing.assert_array_equal(got[name], ref[name], err_msg=name)
  dense = A.dense_grads(q, k, v, do, m.toarray(), d ** -0.5)
  _check(got["dq"], dense[0], dtype, "dq")
  assert A.max_rel_err(got["dk"], dense[1]) > 1e-1


def test_packed_qkv_strides_through_c_abi():
  """q, k, v as strided views of one [B, n, 3, H, D] buffer, read in place by the kernels."""
  rng = np.random.default_rng(10)
  b, n, h, d = 2, 300, 2, 64
  qkv = rng.standard_normal((b, n, 3, h, d)).astype(np.float32)
  m = _random_mask(n, 0.05, 11, symmetric=True)
  tiles = fwn.TileList.from_mask(m)
  buf = torch.from_numpy(qkv).to(DEV)
  out = torch.zeros((b, n, 3, h, d), device=DEV)  # o written in place of the q slot
  desc = nat.AttnDesc(b, n, h, d, nat.F32, d ** -0.5, n * 3 * h * d, 3 * h * d, d)
  lse = torch.empty((b, h, n), device=DEV)
  base = buf.data_ptr()
  step = h * d * 4
  nat.check(nat.lib().fwn_attn_fwd_launch(desc, base, base + step, base + 2 * step, tiles.struct,
                                          out.data_ptr(), lse.data_ptr(), None, 0,
                                          torch.cuda.current_stream().cuda_stream))
  torch.cuda.synchronize()
  got = _np(out[:, :, 0])
  ref = A.dense_attention(qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2], m.toarray(), d ** -0.5)
  _check(got, ref, torch.float32, "out")
  assert (_np(out[:, :, 1:]) == 0).all()  # nothing written outside the o slot


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_deterministic_and_batch_independent(dtype):
  """No atomics: bitwise identical reruns, and each batch element equals its batch-1 run (both
  launches are far below the size at which the library lengthens split-K items)."""
  rng = np.random.default_rng(12)
  b, n, h, d = 3, 400, 2, 128
  q, k, v, do = (rng.standard_normal((b, n, h, d)).astype(np.float32) for _ in range(4))
  tiles = fwn.TileList.from_mask(_random_mask(n, 0.04, 13, symmetric=True))
  r1 = _run(q, k, v, do, tiles, d ** -0.5, dtype)
  r2 = _run(q, k, v, do, tiles, d ** -0.5, dtype)
  for name in r1:
    np.testing.assert_array_equal(r1[name], r2[name])
  one = _run(q[1:2], k[1:2], v[1:2], do[1:2], tiles, d ** -0.5, dtype)
  for name in r1:
    np.testing.assert_array_equal(r1[name][1:2], one[name])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("d", [32, 128])
@pytest.mark.parametrize("max_item_tiles", [1, 3])
def test_split_items_match_dense_reference(max_item_tiles, d, dtype):
  """Blocks cut into several work items (split-K) give the same outputs and gradients: forward
  partials merge by the online-softmax rule, dQ/dK/dV partials by summation. Rows without keys
  inside a split block stay zero."""
  rng = np.random.default_rng(30 + d)
  b, n, h = 2, 900, 2
  q, k, v, do = (_rounded(rng.standard_normal((b, n, h, d)), dtype) for _ in range(4))
  m = _random_mask(n, 0.03, 31, symmetric=True).tolil()
  empty = [5, 300, 777]
  for r in empty:
    m[r, :] = False
    m[:, r] = False
  m = m.tocsr()
  m.eliminate_zeros()
  tp, kb, bits = fwn.build_tile_mask(m)
  tiles = fwn.TileList(tp, kb, bits, n, DEV, max_item_tiles)
  assert tiles.n_split >= len(tp) - 2 and tiles.n_parts > tiles.n_split
  res = _run(q, k, v, do, tiles, d ** -0.5, dtype)
  for name in res:
    assert np.isfinite(res[name]).all(), name
    np.testing.assert_array_equal(res[name][:, empty], 0.0)
  keep = np.setdiff1d(np.arange(n), empty)
  sub = m.toarray()[np.ix_(keep, keep)]
  ref = A.dense_attention(q[:, keep], k[:, keep], v[:, keep], sub, d ** -0.5)
  refs = A.dense_grads(q[:, keep], k[:, keep], v[:, keep], do[:, keep], sub, d ** -0.5)
  for bb in range(b):
    _check(res["out"][bb, keep], ref[bb], dtype, ("out", bb))
    for name, r in zip(("dq", "dk", "dv"), refs):
      _check(res[name][bb, keep], r[bb], dtype, (name, bb))
  # Same log-sum-exp as the unsplit schedule (up to fp32 rounding of the merge).
  whole = fwn.TileList(tp, kb, bits, n, DEV, 10 ** 6)
  assert whole.n_split == 0
  args = [_dev(x, dtype) for x in (q, k, v)]
  _, lse_split = fwn.attention_forward(*args, tiles, d ** -0.5)
  _, lse_whole = fwn.attention_forward(*args, whole, d ** -0.5)
  ls, lw = _np(lse_split), _np(lse_whole)
  assert np.array_equal(np.isinf(ls), np.isinf(lw))
  fin = np.isfinite(lw)
  np.testing.assert_allclose(ls[fin], lw[fin], rtol=0, atol=1e-5)


def test_split_workspace_is_reused_across_calls():
  """One workspace serves consecutive launches on a stream: a second, smaller call with the
  same buffer gives the same result as a fresh one."""
  rng = np.random.default_rng(40)
  n, h, d = 700, 2, 64
  m = _random_mask(n, 0.05, 41, symmetric=True)
  tp, kb, bits = fwn.build_tile_mask(m)
  tiles = fwn.TileList(tp, kb, bits, n, DEV, 2)
  stream = torch.cuda.current_stream().cuda_stream
  outs = []
  for batch in (3, 1):
    q, k, v = (_dev(rng.standard_normal((batch, n, h, d)), torch.float32) for _ in range(3))
    desc = nat.AttnDesc(batch, n, h, d, nat.F32, d ** -0.5, *q.stride()[:3])
    ws = torch.full((tiles.workspace_bytes(nat.AttnDesc(3, n, h, d, nat.F32, d ** -0.5, n * h * d, h * d, d)),),
                    255, dtype=torch.uint8, device=DEV) if not outs else ws
    out = torch.empty_like(q)
    nat.check(nat.lib().fwn_attn_fwd_launch(desc, q.data_ptr(), k.data_ptr(), v.data_ptr(), tiles.struct,
                                            out.data_ptr(), None, ws.data_ptr(), ws.numel(), stream))
    ref, _ = fwn.attention_forward(q, k, v, tiles, d ** -0.5)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_np(out), _np(ref))
    outs.append(out)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("d", [64, 128])
def test_packed_qkv_op_is_bitwise_the_unpacked_op(d, dtype):
  """tiled_flash_attention_qkv reads q, k, v as views of one [B, n, 3, H, D] buffer and writes
  one packed gradient; the kernels see the same values, so outputs and gradients match the
  separate-tensor op bit for bit, and both match the dense oracle."""
  rng = np.random.default_rng(50)
  b, n, h = 2, 500, 2
  qkv_h = _rounded(rng.standard_normal((b, n, 3, h, d)), dtype)
  do_h = _rounded(rng.standard_normal((b, n, h, d)), dtype)
  m = _random_mask(n, 0.04, 51, symmetric=True)
  tiles = fwn.TileList(*fwn.build_tile_mask(m), n, DEV, 2)  # split items as well
  qkv = _dev(qkv_h, dtype, True)
  out = fwn.tiled_flash_attention_qkv(qkv, tiles, scale=d ** -0.5)
  out.backward(_dev(do_h, dtype))
  q, k, v = (_dev(qkv_h[:, :, i], dtype, True) for i in range(3))
  ref = fwn.tiled_flash_attention(q, k, v, tiles, scale=d ** -0.5)
  ref.backward(_dev(do_h, dtype))
  torch.cuda.synchronize()
  np.testing.assert_array_equal(_np(out), _np(ref))
  for i, t in enumerate((q, k, v)):
    np.testing.assert_array_equal(_np(qkv.grad[:, :, i]), _np(t.grad))
  dense = A.dense_attention(qkv_h[:, :, 0], qkv_h[:, :, 1], qkv_h[:, :, 2], m.toarray(), d ** -0.5)
  _check(_np(out), dense, dtype, "out")
  grads = A.dense_grads(qkv_h[:, :, 0], qkv_h[:, :, 1], qkv_h[:, :, 2], do_h, m.toarray(), d ** -0.5)
  for i, name in enumerate(("dq", "dk", "dv")):
    _check(_np(qkv.grad[:, :, i]), grads[i], dtype, name)


def test_tiled_mha_block_matches_unfused_block():
  """TiledMHA (fused projection, in-place kernels) equals the unfused block (separate contiguous
  q, k, v) bit for bit in the output and in every parameter gradient."""
  torch.manual_seed(0)
  b, n, h, d, dm = 1, 700, 2, 64, 128
  m = _random_mask(n, 0.05, 52, symmetric=True)
  tiles = fwn.TileList.from_mask(m, device=DEV)
  block = fwn.TiledMHA(dm, h, d, tiles, device=DEV, dtype=torch.bfloat16)
  x = torch.randn(b, n, dm, device=DEV, dtype=torch.bfloat16)
  grads = []
  outs = []
  for fn in (block.forward, block.forward_unfused):
    block.zero_grad()
    y = fn(x)
    y.float().square().sum().backward()
    outs.append(_np(y))
    grads.append([_np(p.grad) for p in block.parameters()])
  torch.cuda.synchronize()
  np.testing.assert_array_equal(outs[0], outs[1])
  for g0, g1 in zip(*grads):
    np.testing.assert_array_equal(g0, g1)


def test_exp2_based_softmax_accuracy():
  """The softmax uses V_EXP_F32 (2^x) with log2(e) folded into the scale: rows must sum to one and
  the log-sum-exp must match float64 to single-precision accuracy."""
  rng = np.random.default_rng(14)
  n, h, d = 384, 2, 64
  q, k = (3.0 * rng.standard_normal((1, n, h, d)).astype(np.float32) for _ in range(2))
  m = _random_mask(n, 0.2, 15, symmetric=True)
  tiles = fwn.TileList.from_mask(m)
  ones = np.ones((1, n, h, d), np.float32)
  out, lse = fwn.attention_forward(_dev(q, torch.float32), _dev(k, torch.float32), _dev(ones, torch.float32),
                                   tiles, d ** -0.5)
  np.testing.assert_allclose(_np(out), 1.0, rtol=0, atol=4e-6)
  ref = A.dense_lse(q, k, m.toarray(), d ** -0.5)
  np.testing.assert_allclose(_np(lse), ref, rtol=2e-6, atol=2e-6)


def _extreme_logit_case(d, seed):
  """Three row groups of 192 (n = 576, a ragged last block): rows 0-191 take keys 0-191, whose
  logits are O(1); rows 192-383 take keys 192-383, whose logits are about +100 (natural units),
  plus the keys of 0-191 within 100 rows; rows 384-575 take keys 384-575 only, whose logits are
  about -100. Channel 0 carries the offsets (q = 1, k = +-100 / scale rounded to bf16, so that
  every precision holds it exactly), the other channels are standard normal. Every masked key of the first and last groups has a logit far
  above the valid ones: had it entered a row's reference max, exp2 of the valid logits would
  underflow (2^-144 and below) and the row would come out zero or NaN. The middle rows' max
  jumps by about 144 (log2 units) between tiles, so the running sums are rescaled by factors that
  underflow."""
  rng = np.random.default_rng(seed)
  n, g = 576, 192
  scale = d ** -0.5
  rows, cols = [], []
  for i in range(n):
    grp = i // g
    lo, hi = (i - 100, i + 40) if grp == 1 else (i - 60, i + 60)
    ks = np.arange(max(lo, 0 if grp != 2 else 2 * g), min(hi, (grp + 1) * g - 1) + 1)
    if grp == 0:
      ks = ks[ks < g]
    rows.extend([i] * len(ks))
    cols.extend(ks.tolist())
  m = sparse.csr_matrix((np.ones(len(rows), bool), (rows, cols)), shape=(n, n))
  q = rng.standard_normal((1, n, 2, d))
  k = rng.standard_normal((1, n, 2, d))
  q[..., 0] = 1.0
  k[:, :g, :, 0] = 0.0
  off = float(torch.tensor(100.0 / scale).to(torch.bfloat16))
  k[:, g:2 * g, :, 0] = off
  k[:, 2 * g:, :, 0] = -off
  v, do = (rng.standard_normal((1, n, 2, d)) for _ in range(2))
  return m, scale, q, k, v, do


def _grad_rounding_bounds(q, k, v, do, out, dense, scale):
  """Per element of dq and of dk, float64 sums that bound their rounding error:
  dq_i: scale sum_j (|dS_ij| + P_ij |o_i| . |do_i|) |k_j|;  dk_j: scale sum_i (same) |q_i|.
  dq = scale sum_j dS_ij k_j and dk = scale sum_i dS_ij q_i, with dS = P (dP - delta) and
  delta = o . do: a relative error u in each dS_ij (dS rounded to bf16 for its products with K
  and Q) and one of u times |o_i| . |do_i| in delta_i (o is the rounded forward output) move dq
  and dk by at most u times these sums. Where sum_j dS_ij k_j cancels (sum_j dS_ij = 0: keys
  whose logits share a large offset, or rows with very few keys) or dP - delta does (few keys),
  the error is set by these sums, not by the gradients themselves."""
  p = A._dense_probs(q, k, dense, scale)
  q64, k64, v64, do64, o64 = (x.astype(np.float64) for x in (q, k, v, do, out))
  dp = np.einsum("bnhd,bmhd->bhnm", do64, v64)
  ds = p * (dp - (dp * p).sum(-1, keepdims=True))
  od = np.einsum("bnhd,bnhd->bhn", np.abs(do64), np.abs(o64))
  w = np.abs(ds) + p * od[..., None]
  bq = scale * np.einsum("bhnm,bmhd->bnhd", w, np.abs(k64))
  bk = scale * np.einsum("bhnm,bnhd->bmhd", w, np.abs(q64))
  return bq, bk


@pytest.mark.parametrize("case", ["bf16", "f32", "bf16x3"])
@pytest.mark.parametrize("d", [64, 128])
def test_extreme_logits_and_masked_giants(d, case):
  """Rows whose valid logits are all near -100, rows whose masked keys carry logits up to +100
  above their valid ones, and rows whose max jumps by +100 halfway (_extreme_logit_case):
  forward, log-sum-exp and gradients (bf16: the dS exchange) against the dense float64 oracle.
  out, dk and dv meet the usual bars in bf16; in float32 the logits of magnitude 100 carry
  rounding of about 1e-5 in absolute terms (one unit in the last place of 100 is 7.6e-6, and the
  kernel scales and sums them), which enters each probability as a relative error of that size:
  bars 4e-5 (rms) and 2e-4 (max). dq = scale sum_j dS_ij k_j cancels (channel 0 of k carries the
  +-100 offsets, and sum_j dS_ij = 0), so it is held to the rounding bound of that sum
  (_grad_rounding_bounds) with u = 2^-7 in bf16 (twice bf16's unit roundoff) and 2^-14 in float32
  (float32's unit roundoff times the about 1,000 terms an element sums). bf16x3 (float32 tensors,
  products from bf16 parts) is held to the float32 bars: the offsets are exact in bf16, so the
  split leaves them whole, and the other channels are of order one."""
  print(f"extreme logits d={d} {case}", flush=True)
  dtype = torch.bfloat16 if case == "bf16" else torch.float32
  precision = "bf16x3" if case == "bf16x3" else "native"
  m, scale, q, k, v, do = _extreme_logit_case(d, 60 + d)
  q, k, v, do = (_rounded(x, dtype) for x in (q, k, v, do))
  tiles = fwn.TileList.from_mask(m)
  tiles_t = fwn.TileList.from_mask(m.T.tocsr())
  out, lse = fwn.attention_forward(*(_dev(x, dtype) for x in (q, k, v)), tiles, scale, precision=precision)
  qt, kt, vt = (_dev(x, dtype, True) for x in (q, k, v))
  res = fwn.tiled_flash_attention(qt, kt, vt, tiles, scale=scale, tiles_t=tiles_t, precision=precision)
  res.backward(_dev(do, dtype))
  got = {"out": _np(res), "dq": _np(qt.grad), "dk": _np(kt.grad), "dv": _np(vt.grad)}
  torch.cuda.synchronize()
  dense = m.toarray()
  ref_lse = A.dense_lse(q, k, dense, scale)
  assert np.isfinite(_np(lse)).all() and np.isfinite(got["out"]).all()
  # lse sits near -100, 0 and +100 in the three groups; its error is the logits' rounding.
  np.testing.assert_allclose(_np(lse), ref_lse, rtol=0, atol=2e-3 if dtype == torch.bfloat16 else 1e-4)
  np.testing.assert_array_equal(_np(out), got["out"])
  rms, mx = (5e-3, 3e-2) if dtype == torch.bfloat16 else (4e-5, 2e-4)
  ref_dq, ref_dk, ref_dv = A.dense_grads(q, k, v, do, dense, scale)
  for name, r in (("out", A.dense_attention(q, k, v, dense, scale)), ("dk", ref_dk), ("dv", ref_dv)):
    assert np.isfinite(got[name]).all(), name
    rr, mr = A.rel_rms(got[name], r), A.max_rel_err(got[name], r)
    print(f"  {name}: rel rms {rr:.2e}, max {mr:.2e}", flush=True)
    assert rr <= rms and mr <= mx, (name, rr, mr)
  assert np.isfinite(got["dq"]).all()
  bound = _grad_rounding_bounds(q, k, v, do, got["out"], dense, scale)[0]
  u = 2.0 ** -7 if dtype == torch.bfloat16 else 2.0 ** -14
  ratio = np.abs(got["dq"] - ref_dq) / (u * bound + 1e-30)
  print(f"  dq: rel rms {A.rel_rms(got['dq'], ref_dq):.2e}, error / bound max {ratio.max():.3f}", flush=True)
  assert ratio.max() <= 1.0, ratio.max()


def test_reference_keywords_give_the_same_result():
  """A call written for the reference's signature (pallas_attn.py:317-320: strict_fp32, block
  sizes, Triton tuning values) runs the same kernels: bit-identical outputs and gradients."""
  rng = np.random.default_rng(12)
  n, h, d = 300, 2, 64
  q, k, v, do = (rng.standard_normal((1, n, h, d)).astype(np.float32) for _ in range(4))
  tiles = fwn.TileList.from_mask(_random_mask(n, 0.05, 13, symmetric=True))
  res = []
  for kw in ({}, dict(strict_fp32=True, block_q=128, block_k=128, num_warps=4, num_stages=1, bwd_num_warps=4,
                      bwd_split=2, interpret=False)):
    qt, kt, vt = (_dev(x, torch.float32, True) for x in (q, k, v))
    out = fwn.tiled_flash_attention(qt, kt, vt, tiles, scale=d ** -0.5, **kw)
    out.backward(_dev(do, torch.float32))
    res.append([_np(t) for t in (out, qt.grad, kt.grad, vt.grad)])
  torch.cuda.synchronize()
  for a, b in zip(*res):
    np.testing.assert_array_equal(a, b)


def _tiled_mha_reference(x, wqkv, wf, bf, mask, heads, key_size):
  """The reference's tiled_mha (patch.py:165-177) in float64 on the CPU: q, k, v projections
  [batch, n, heads, key_size] (the fused weight's rows are q, k, v in turn, each head-major), masked
  softmax attention with scale key_size**-0.5 (masked logits -inf), reshape to
  [batch, n, heads * key_size], then the mha_final projection with bias."""
  b, n, _ = x.shape
  q, k, v = (x @ w.T for w in wqkv.split(heads * key_size))
  q, k, v = (t.view(b, n, heads, key_size).transpose(1, 2) for t in (q, k, v))
  s = (q @ k.transpose(-1, -2)) * key_size ** -0.5
  p = torch.softmax(s.masked_fill(~mask, float("-inf")), dim=-1)
  o = (p @ v).transpose(1, 2).reshape(b, n, heads * key_size)
  return o @ wf.T + bf


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_tiled_mha_block_matches_reference_composition(dtype):
  """TiledMHA (the reference's tiled_mha caller, patch.py:165-177) against that composition
  restated in float64 autograd on the CPU with the block's own weights (rounded to dtype): the
  output and the gradients of the input and of every weight, max rel RMS 1e-5 (float32) /
  5e-3 (bf16)."""
  print(f"tiled_mha composition {dtype}", flush=True)
  torch.manual_seed(1)
  b, n, h, d, dm = 2, 600, 2, 64, 96
  m = _random_mask(n, 0.05, 53, symmetric=True)
  tiles = fwn.TileList.from_mask(m, device=DEV)
  block = fwn.TiledMHA(dm, h, d, tiles, device=DEV, dtype=dtype, precision="native")
  with torch.no_grad():
    block.final.bias.normal_(0, 0.5)
  x = torch.randn(b, n, dm, device=DEV, dtype=dtype, requires_grad=True)
  g = torch.randn(b, n, dm, device=DEV, dtype=dtype)
  y = block(x)
  y.backward(g)
  torch.cuda.synchronize()
  ws = [p.detach().double().cpu().requires_grad_(True) for p in (block.qkv.weight, block.final.weight, block.final.bias)]
  xr = x.detach().double().cpu().requires_grad_(True)
  ref = _tiled_mha_reference(xr, *ws, torch.from_numpy(m.toarray()), h, d)
  ref.backward(g.double().cpu())
  pairs = [("out", y, ref), ("dx", x.grad, xr.grad), ("dWqkv", block.qkv.weight.grad, ws[0].grad),
           ("dWfinal", block.final.weight.grad, ws[1].grad), ("dbias", block.final.bias.grad, ws[2].grad)]
  for what, got, want in pairs:
    got, want = got.detach().double().cpu().numpy(), want.detach().numpy()
    assert A.rel_rms(got, want) <= TOL[dtype], (what, A.rel_rms(got, want))
