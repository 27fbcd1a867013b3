"""GPU parity at model scale: the refinement-6 mesh (40,962 nodes), configurations 2-5 of
BASELINE.json and the reference's own benchmark shape (scripts/attn_bench.py:23, 115-119: 32-hop,
Hilbert order, 6 heads x 128).

The float64 oracle (oracle.attention.block_attention) is exact at whole 128-row blocks (out, lse,
dq) and whole 128-key blocks (dk, dv). Each test checks blocks the launched split-K schedule cuts
into several items (their partial results go through the combine pass), blocks it does not, and
the ragged last block 320 (40,962 = 320 * 128 + 2), plus size-independent identities over all
nodes: rows of P sum to one, so sum_j dV_j = sum_i dO_i, and rows of dS sum to zero, so
sum_j dK_j = 0.
"""
import numpy as np
import pytest
import torch

import faster_weathernext_amd as fwn
from faster_weathernext_amd import _native as nat
from faster_weathernext_amd import hip_attn
from gpu_helpers import check, check_blocks, dev, host, rounded, run
from oracle import attention as A

pytestmark = pytest.mark.gpu
BF16, F32 = torch.bfloat16, torch.float32
SCALE = 128 ** -0.5
LAST = 320  # ragged last block of the refinement-6 mesh


@pytest.fixture(scope="module")
def r6():
  """k-hop masks of the refinement-6 mesh, in subdivision order or permuted to Hilbert order."""
  cache = {}

  def get(k, hilbert=False):
    if (k, hilbert) not in cache:
      mask, _, _, perm = fwn.mesh_mask(6, k, reorder=hilbert)
      cache[(k, hilbert)] = mask[perm][:, perm].tocsr() if hilbert else mask
    return cache[(k, hilbert)]

  return get


def _inputs(seeds, n, heads, dtype, sigma=1.0, grads=True):
  """q, k, v (N(0, sigma)) then dO (N(0, 1)) per member from PCG64 seed m, rounded to dtype."""
  out = [[], [], [], []]
  for m in seeds:
    rng = np.random.default_rng(m)
    for i in range(4 if grads else 3):
      x = rng.standard_normal((1, n, heads, 128)) * (sigma if i < 3 else 1.0)
      out[i].append(rounded(x, dtype))
  return [np.concatenate(x) if x else None for x in out]


def _split_blocks(tl, batch, heads):
  return set(int(b) for b in tl.schedule_for(batch, heads).split_host[:, 0])


def _identities(res, do):
  """sum_j dV_j = sum_i dO_i and sum_j dK_j = 0 over all nodes, per member and head."""
  scale_dv = np.abs(do).sum(1)
  np.testing.assert_allclose(res["dv"].astype(np.float64).sum(1), do.astype(np.float64).sum(1),
                             rtol=0, atol=float(5e-3 * scale_dv.max()))
  assert np.abs(res["dk"].astype(np.float64).sum(1)).max() <= 5e-3 * np.abs(res["dk"]).sum(1).max()


def _same_to_combine_rounding(a, b, what):
  """Two schedules of the same bf16 call: the split-K combine sums float32 partials in another
  order, so an element may differ by one bf16 rounding step."""
  for name in a:
    x, y = a[name].astype(np.float64), b[name].astype(np.float64)
    np.testing.assert_allclose(x, y, rtol=0, atol=float(2 ** -7 * np.abs(y).max()), err_msg=f"{what} {name}")
    assert A.rel_rms(x, y) <= 2e-3, (what, name, A.rel_rms(x, y))


@pytest.mark.parametrize("sigma", [128 ** -0.5, 1.0])
def test_c2_fp32_forward(r6, sigma):
  """Configuration 2: 8-hop mask in subdivision order, 4 heads x 128, float32 MFMA, forward
  (sigma = 128^-1/2 as the config states, and 1 for a sharper check)."""
  mask = r6(8)
  n = mask.shape[0]
  q, k, v, _ = _inputs([0], n, 4, F32, sigma, grads=False)
  tiles = fwn.TileList.from_mask(mask)
  assert 0 in _split_blocks(tiles, 1, 4)  # block 0 holds all 320 column tiles
  out, lse = fwn.attention_forward(*(dev(x, F32) for x in (q, k, v)), tiles, SCALE)
  ref = A.block_attention(q, k, v, np.zeros_like(q), mask, SCALE, row_blocks=[0, 160, LAST])
  check(host(out)[:, ref["rows"]], ref["out"], F32, "out")
  np.testing.assert_allclose(host(lse)[:, :, ref["rows"]], ref["lse"], rtol=0, atol=1e-5)


def test_c3_bf16_forward_backward_whole_blocks(r6):
  """Configuration 3: 16-hop mask, 4 heads x 128, bf16 with fp32 accumulation, fwd + bwd. Rows of
  blocks 0 (320 tiles, five items), 77 (67 tiles, two items) and 320; every key of blocks 77
  (split), 200 (48 tiles, one item) and 320."""
  mask = r6(16)
  n = mask.shape[0]
  q, k, v, do = _inputs([0], n, 4, BF16)
  tiles = fwn.TileList.from_mask(mask)
  split = _split_blocks(tiles, 1, 4)
  assert {0, 77} <= split and 200 not in split and LAST not in split
  res = run(q, k, v, do, tiles, SCALE, BF16)
  ref = A.block_attention(q, k, v, do, mask, SCALE, row_blocks=[0, 77, LAST], key_blocks=[77, 200, LAST])
  check_blocks(res, ref, BF16, "c3")
  _identities(res, do)


def test_c4_bf16_ensemble_forward_backward(r6):
  """Configuration 4: 8 members sharing one 8-hop tile list, bf16, fwd + bwd; member m drawn from
  seed m. The 8-member launch (10,272 jobs) runs the 128-tile schedule, which still splits blocks
  0-4. Members 0 and 7 are checked against the oracle at rows of blocks 4 and 320 and keys of
  blocks 4 (161 tiles, split), 200 and 320; the whole batch against the 64-tile schedule to the
  rounding of the combine; and, with the cap pinned, member 7 alone equals member 7 in the batch
  bit for bit."""
  mask = r6(8)
  n = mask.shape[0]
  q, k, v, do = _inputs(range(8), n, 4, BF16)
  tiles = fwn.TileList.from_mask(mask)
  assert tiles.item_cap_for(8, 4) == hip_attn.WIDE_ITEM_TILES
  assert tiles.item_cap_for(1, 4) == nat.ITEM_TILES
  assert _split_blocks(tiles, 8, 4) == {0, 1, 2, 3, 4}
  res = run(q, k, v, do, tiles, SCALE, BF16)
  for m in (0, 7):
    ref = A.block_attention(q[m:m + 1], k[m:m + 1], v[m:m + 1], do[m:m + 1], mask, SCALE, row_blocks=[4, LAST],
                            key_blocks=[4, 200, LAST])
    check_blocks({name: x[m:m + 1] for name, x in res.items()}, ref, BF16, ("member", m))
  _identities(res, do)
  pinned = fwn.TileList.from_mask(mask, max_item_tiles=nat.ITEM_TILES)
  batch64 = run(q, k, v, do, pinned, SCALE, BF16)
  _same_to_combine_rounding(res, batch64, "c4 128- vs 64-tile items")
  one = run(q[7:8], k[7:8], v[7:8], do[7:8], pinned, SCALE, BF16)
  for name in one:
    np.testing.assert_array_equal(batch64[name][7:8], one[name], err_msg=name)


def test_c5_attention_shape_bf16_forward_backward(r6):
  """The reference benchmark's attention (scripts/attn_bench.py:23, 115-119) and WN2's layer
  shape: 32-hop mask in Hilbert order, 6 heads x 128, bf16, fwd + bwd. A third of its live 32 x 32
  groups are fully valid and take the unmasked path. The call (1,926 jobs) launches 128-tile items,
  which split nothing; the 64-tile schedule splits 33 blocks (119, the longest at 97 tiles, among
  them) and must agree to the rounding of the combine. Rows of blocks 119 and 320, every key of
  blocks 119, 200 (94 tiles) and 320."""
  mask = r6(32, hilbert=True)
  n = mask.shape[0]
  q, k, v, do = _inputs([0], n, 6, BF16)
  tiles = fwn.TileList.from_mask(mask)
  assert tiles.item_cap_for(1, 6) == hip_attn.WIDE_ITEM_TILES and not _split_blocks(tiles, 1, 6)
  full = np.unpackbits((tiles.groups_host >> 16).astype("<u2").view(np.uint8)).sum()
  assert full > 0.25 * np.unpackbits((tiles.groups_host & 0xFFFF).astype("<u2").view(np.uint8)).sum()
  res = run(q, k, v, do, tiles, SCALE, BF16)
  ref = A.block_attention(q, k, v, do, mask, SCALE, row_blocks=[119, LAST], key_blocks=[119, 200, LAST])
  check_blocks(res, ref, BF16, "c5")
  _identities(res, do)
  pinned = fwn.TileList.from_mask(mask, max_item_tiles=nat.ITEM_TILES)
  assert {119, 200} <= _split_blocks(pinned, 1, 6) and len(_split_blocks(pinned, 1, 6)) == 33
  _same_to_combine_rounding(res, run(q, k, v, do, pinned, SCALE, BF16), "c5 128- vs 64-tile items")


def test_c5_attention_shape_fp32_forward_backward(r6):
  """The same shape at full precision (fp32 MFMA; the reference's strict_fp32, and tighter than its
  "highest" 3xTF32 mode, pallas_attn.py:336-347): forward and backward within rel RMS 1e-5 and the
  reference's max-relative bar, lse within 1e-5, at rows of blocks 119, 200 and 320 and every key of
  blocks 119, 200 and 320 (bench.py --workload c5f32 times this call)."""
  mask = r6(32, hilbert=True)
  n = mask.shape[0]
  q, k, v, do = _inputs([0], n, 6, F32)
  tiles = fwn.TileList.from_mask(mask)
  res = run(q, k, v, do, tiles, SCALE, F32)
  ref = A.block_attention(q, k, v, do, mask, SCALE, row_blocks=[119, 200, LAST], key_blocks=[119, 200, LAST])
  check_blocks(res, ref, F32, "c5 fp32")
  _, lse = fwn.attention_forward(*(dev(x, F32) for x in (q, k, v)), tiles, SCALE)
  np.testing.assert_allclose(host(lse)[:, :, ref["rows"]], ref["lse"], rtol=0, atol=1e-5)


def test_hilbert_reordering_is_exact_up_to_rounding(r6):
  """Attention on Hilbert-permuted nodes with the permuted mask, un-permuted, equals attention in
  subdivision order (patch.py:275-292 relies on this)."""
  mask = r6(8)
  _, _, _, perm = fwn.mesh_mask(6, 8, reorder=True)
  n = mask.shape[0]
  rng = np.random.default_rng(5)
  q, k, v = (rng.standard_normal((1, n, 2, 64)).astype(np.float32) for _ in range(3))
  plain = fwn.TileList.from_mask(mask)
  hil = fwn.TileList.from_mask(mask, perm)
  assert hil.n_tiles < plain.n_tiles
  a, _ = fwn.attention_forward(*(dev(x, F32) for x in (q, k, v)), plain, 64 ** -0.5, with_lse=False)
  b, _ = fwn.attention_forward(*(dev(x[:, perm], F32) for x in (q, k, v)), hil, 64 ** -0.5, with_lse=False)
  inv = np.argsort(perm)
  assert A.rel_rms(host(b)[:, inv], host(a)) <= 1e-6
