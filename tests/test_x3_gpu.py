"""GPU parity of the split-precision forward (precision "bf16x3", FWN_PREC_BF16X3): float32
tensors whose products are formed from bf16 parts, hi*hi + hi*lo + lo*hi.

Each operand carries about 17 significant bits (hi + lo), so a logit s = q.k carries an absolute
error of about 2^-17 |q||k|: the error grows with the logits' magnitude. With inputs of standard
deviation <= 1 (every configuration of BASELINE.json) the outputs stay within its float32 bar,
rel RMS <= 1e-5 per output tensor against the float64 oracle on the same float32 inputs, and
max|got - ref| / max|ref| (the reference's unit-test metric, tests/test_pallas_kernel.py:54, 98)
within 2e-5. With sigma = 4 (logits of standard deviation 16) the bar is rel RMS 3e-5 and
max 1e-4; TF32 dots, the reference's default (pallas_attn.py:342-343), are about 30x coarser.
The backward runs in bf16x3 too (the dS exchange: dK/dV writes dS as hi and lo parts, dQ reads
them); lists that are not exact transposes take the recomputing IEEE float32 backward.
"""
import numpy as np
import pytest
import torch
from scipy import sparse

import faster_weathernext_amd as fwn
from faster_weathernext_amd import hip_attn
from gpu_helpers import dev, host, random_mask
from oracle import attention as A

pytestmark = pytest.mark.gpu
F32 = torch.float32
X3 = "bf16x3"


def check(got, ref, what, rms=1e-5, mx=2e-5):
  rr, mr = A.rel_rms(got, ref), A.max_rel_err(got, ref)
  assert rr <= rms and mr <= mx, (what, rr, mr)


def _fwd(q, k, v, tiles, scale, precision=X3):
  out, lse = fwn.attention_forward(dev(q, F32), dev(k, F32), dev(v, F32), tiles, scale, precision=precision)
  torch.cuda.synchronize()
  return host(out), host(lse)


def test_c1_golden():
  g = np.load(__file__.replace("test_x3_gpu.py", "golden/c1_r3_2hop.npz"))
  n = g["q"].shape[1]
  mask = sparse.csr_matrix((np.ones(len(g["indices"]), bool), g["indices"], g["indptr"]), shape=(n, n))
  tiles = fwn.TileList.from_mask(mask)
  scale = float(g["scale"])
  out, lse = _fwd(g["q"], g["k"], g["v"], tiles, scale)
  check(out, g["out"], "out")
  np.testing.assert_allclose(lse, g["lse"], rtol=0, atol=2e-5)


@pytest.mark.parametrize("d", [32, 64, 128])
@pytest.mark.parametrize("cap", [None, 1, 3])
@pytest.mark.parametrize("sigma", [1.0, 4.0])
def test_random_masks_match_dense_oracle(d, cap, sigma):
  """The reference's random-mask generator (tests/test_pallas_kernel.py:72-99: n = 300, density
  0.05 plus the identity) at every built head_dim, whole and split work items; sigma = 4 gives
  peaked rows, where a product's rounding moves the softmax the most."""
  rng = np.random.default_rng(2)
  n, h = 300, 2
  q, k, v = (rng.standard_normal((2, n, h, d)).astype(np.float32) * s for s in (sigma, sigma, 1.0))
  mask = random_mask(n, 0.05, 3)
  tiles = fwn.TileList.from_mask(mask, max_item_tiles=cap)
  scale = d ** -0.5
  out, lse = _fwd(q, k, v, tiles, scale)
  dense = mask.toarray()
  sharp = sigma > 1
  check(out, A.dense_attention(q, k, v, dense, scale), "out", 3e-5 if sharp else 1e-5, 1e-4 if sharp else 2e-5)
  np.testing.assert_allclose(lse, A.dense_lse(q, k, dense, scale), rtol=3e-5 if sharp else 0, atol=2e-5)


def test_rows_without_keys_and_partial_tiles():
  """A mask with empty rows (output 0, as the native kernels), a ragged last block (n = 200) and
  single-element tiles."""
  n, h, d = 200, 1, 64
  rng = np.random.default_rng(5)
  q, k, v = (rng.standard_normal((1, n, h, d)).astype(np.float32) for _ in range(3))
  dense = np.zeros((n, n), bool)
  dense[np.arange(0, n, 3), (np.arange(0, n, 3) * 7) % n] = True
  dense[150:, :10] = True
  mask = sparse.csr_matrix(dense)
  tiles = fwn.TileList.from_mask(mask)
  out, _ = _fwd(q, k, v, tiles, d ** -0.5)
  native, _ = _fwd(q, k, v, tiles, d ** -0.5, precision="native")
  empty = ~dense.any(1)
  assert np.all(out[:, empty] == 0) and np.all(native[:, empty] == 0)
  ref = A.dense_attention(q, k, v, dense, d ** -0.5)
  check(out[:, ~empty], ref[:, ~empty], "out")


def test_c2_forward_model_scale():
  """Configuration 2 (refinement 6, 8-hop, subdivision order, 4 heads x 128, float32) through the
  split-precision forward: rows of blocks 0 (split into several items), 160 and the ragged 320,
  for sigma = 128^-1/2 (the config) and 1."""
  mask, _, _, _ = fwn.mesh_mask(6, 8)
  n = mask.shape[0]
  tiles = fwn.TileList.from_mask(mask)
  for sigma in (128 ** -0.5, 1.0):
    rng = np.random.default_rng(0)
    q, k, v = (rng.standard_normal((1, n, 4, 128)).astype(np.float32) * sigma for _ in range(3))
    out, lse = _fwd(q, k, v, tiles, 128 ** -0.5)
    ref = A.block_attention(q, k, v, np.zeros_like(q), mask, 128 ** -0.5, row_blocks=[0, 160, 320])
    check(out[:, ref["rows"]], ref["out"], ("out", sigma))
    np.testing.assert_allclose(lse[:, :, ref["rows"]], ref["lse"], rtol=0, atol=1e-5)


def _grads(q, k, v, do, tiles, scale, tiles_t=None):
  qt, kt, vt = (dev(x, F32, True) for x in (q, k, v))
  out = fwn.tiled_flash_attention(qt, kt, vt, tiles, scale=scale, precision=X3, tiles_t=tiles_t)
  out.backward(dev(do, F32))
  torch.cuda.synchronize()
  return {"out": host(out), "dq": host(qt.grad), "dk": host(kt.grad), "dv": host(vt.grad)}


def test_c1_golden_gradients():
  g = np.load(__file__.replace("test_x3_gpu.py", "golden/c1_r3_2hop.npz"))
  n = g["q"].shape[1]
  mask = sparse.csr_matrix((np.ones(len(g["indices"]), bool), g["indices"], g["indptr"]), shape=(n, n))
  res = _grads(g["q"], g["k"], g["v"], g["do"], fwn.TileList.from_mask(mask), float(g["scale"]))
  for name in ("out", "dq", "dk", "dv"):
    check(res[name], g[name], name)


@pytest.mark.parametrize("d", [32, 64, 128])
@pytest.mark.parametrize("cap", [None, 1, 3])
def test_backward_matches_dense_oracle(d, cap):
  """The bf16x3 backward (dS exchange) on a symmetric random mask, batch 2, whole and split work
  items (split blocks go through the combine passes), against the float64 gradients."""
  rng = np.random.default_rng(0)
  n, h = 300, 2
  q, k, v, do = (rng.standard_normal((2, n, h, d)).astype(np.float32) for _ in range(4))
  mask = random_mask(n, 0.05, 1, symmetric=True)
  tiles = fwn.TileList.from_mask(mask, max_item_tiles=cap)
  res = _grads(q, k, v, do, tiles, d ** -0.5)
  dense = mask.toarray()
  check(res["out"], A.dense_attention(q, k, v, dense, d ** -0.5), "out")
  for name, ref in zip(("dq", "dk", "dv"), A.dense_grads(q, k, v, do, dense, d ** -0.5)):
    check(res[name], ref, name)


@pytest.mark.parametrize("exchange", [True, False])
def test_non_symmetric_mask_with_its_transposed_list(exchange, monkeypatch):
  """A non-symmetric mask with its transposed list (the reference's tiles_t): the bf16x3 dS
  exchange walks the transposed list in dK/dV and the forward list in dQ. With the exchange off
  the backward is the recomputing IEEE float32 one. Both within the bar."""
  monkeypatch.setattr(hip_attn, "DS_EXCHANGE", exchange)
  rng = np.random.default_rng(3)
  n, h, d = 280, 2, 64
  q, k, v, do = (rng.standard_normal((1, n, h, d)).astype(np.float32) for _ in range(4))
  mask = random_mask(n, 0.06, 5)
  tiles, tiles_t = fwn.TileList.from_mask(mask), fwn.TileList.from_mask(mask.T.tocsr())
  assert tiles.ds_map(tiles_t, 32) is not None
  res = _grads(q, k, v, do, tiles, d ** -0.5, tiles_t=tiles_t)
  dense = mask.toarray()
  check(res["out"], A.dense_attention(q, k, v, dense, d ** -0.5), "out")
  for name, ref in zip(("dq", "dk", "dv"), A.dense_grads(q, k, v, do, dense, d ** -0.5)):
    check(res[name], ref, name)


def test_c3_mask_float32_model_scale():
  """The 16-hop refinement-6 mask (configuration 3's), float32 tensors in bf16x3, 2 heads x 128,
  fwd + bwd: rows of blocks 0, 77 and 320 and every key of blocks 77, 200 and 320 against the
  exact block oracle, plus sum_j dV_j = sum_i dO_i and sum_j dK_j = 0 over all nodes."""
  mask, _, _, _ = fwn.mesh_mask(6, 16)
  n = mask.shape[0]
  rng = np.random.default_rng(0)
  q, k, v, do = (rng.standard_normal((1, n, 2, 128)).astype(np.float32) for _ in range(4))
  res = _grads(q, k, v, do, fwn.TileList.from_mask(mask), 128 ** -0.5)
  ref = A.block_attention(q, k, v, do, mask, 128 ** -0.5, row_blocks=[0, 77, 320], key_blocks=[77, 200, 320])
  check(res["out"][:, ref["rows"]], ref["out"], "out")
  check(res["dq"][:, ref["rows"]], ref["dq"], "dq")
  check(res["dk"][:, ref["keys"]], ref["dk"], "dk")
  check(res["dv"][:, ref["keys"]], ref["dv"], "dv")
  np.testing.assert_allclose(res["dv"].astype(np.float64).sum(1), do.astype(np.float64).sum(1), rtol=0,
                             atol=float(1e-4 * np.abs(do).sum(1).max()))
  assert np.abs(res["dk"].astype(np.float64).sum(1)).max() <= 1e-4 * np.abs(res["dk"]).sum(1).max()


def test_packed_qkv_strided_views():
  """q, k, v as strided views of one [B, n, 3, H, D] buffer (the split pass reads them in place)
  give the same output as contiguous copies, bit for bit."""
  rng = np.random.default_rng(4)
  b, n, h, d = 2, 260, 3, 32
  qkv = dev(rng.standard_normal((b, n, 3, h, d)), F32)
  mask = random_mask(n, 0.08, 7, symmetric=True)
  tiles = fwn.TileList.from_mask(mask)
  packed = fwn.tiled_flash_attention_qkv(qkv, tiles, scale=d ** -0.5, precision=X3)
  q, k, v = (qkv[:, :, i].contiguous() for i in range(3))
  plain = fwn.tiled_flash_attention(q, k, v, tiles, scale=d ** -0.5, precision=X3)
  torch.cuda.synchronize()
  assert torch.equal(packed, plain)


def test_more_accurate_than_bf16_and_close_to_native():
  """bf16x3 sits between the bf16 path and IEEE float32: against the float64 oracle its error is
  far below bf16's and within a small factor of the float32 kernel's."""
  rng = np.random.default_rng(8)
  n, h, d = 300, 2, 128
  q, k, v = (rng.standard_normal((1, n, h, d)).astype(np.float32) for _ in range(3))
  mask = random_mask(n, 0.2, 9, symmetric=True)
  tiles = fwn.TileList.from_mask(mask)
  ref = A.dense_attention(q, k, v, mask.toarray(), d ** -0.5)
  x3, _ = _fwd(q, k, v, tiles, d ** -0.5)
  native, _ = _fwd(q, k, v, tiles, d ** -0.5, precision="native")
  bf, _ = fwn.attention_forward(*(dev(x, torch.bfloat16) for x in (q, k, v)), tiles, d ** -0.5)
  e_x3, e_nat, e_bf = A.rel_rms(x3, ref), A.rel_rms(native, ref), A.rel_rms(host(bf), ref)
  assert e_x3 <= 1e-5 and e_x3 * 50 < e_bf and e_x3 < 30 * max(e_nat, 1e-7), (e_x3, e_nat, e_bf)


def test_c5_attention_shape_forward_backward():
  """The reference benchmark's attention shape (scripts/attn_bench.py:23, 115-119: 32-hop mask
  in Hilbert order, 6 heads x 128, fwd + bwd) with float32 tensors in bf16x3 (bench.py
  --workload c5f32 --precision bf16x3 times this call): rows of blocks 119, 200 and 320 and every
  key of blocks 119, 200 and 320 against the exact block oracle, within the float32 bar."""
  mask, _, _, perm = fwn.mesh_mask(6, 32, reorder=True)
  mask = mask[perm][:, perm].tocsr()
  n = mask.shape[0]
  rng = np.random.default_rng(0)
  q, k, v, do = (rng.standard_normal((1, n, 6, 128)).astype(np.float32) for _ in range(4))
  res = _grads(q, k, v, do, fwn.TileList.from_mask(mask), 128 ** -0.5)
  ref = A.block_attention(q, k, v, do, mask, 128 ** -0.5, row_blocks=[119, 200, 320], key_blocks=[119, 200, 320])
  check(res["out"][:, ref["rows"]], ref["out"], "out")
  check(res["dq"][:, ref["rows"]], ref["dq"], "dq")
  check(res["dk"][:, ref["keys"]], ref["dk"], "dk")
  check(res["dv"][:, ref["keys"]], ref["dv"], "dv")
