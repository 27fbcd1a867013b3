"""GPU parity of the 16-key dK/dV kernels' skipping paths at head_dim 128 (float32 tensors, IEEE
fp32 and bf16x3 products), on a mask designed so that each path is taken.

A dK/dV unit is one wave's 16 keys x one 32-query group of a tile of the transposed list. The
designed tile holds a unit valid only in its first 16-query half, one valid only in its second
half (the IEEE fp32 kernel skips the other half's MFMAs), a 32 x 32 group in which only the first
16 keys have a valid element (the other wave writes zeros for its share of the float32 exchange's
unit), a full unit, a sparse unit with both halves and a single element. The reference's kernel
has no such paths (pallas_attn.py:187-215 computes every element of every live tile); the bar is
the dense float64 oracle's, as for every other mask.
"""
import numpy as np
import pytest
import torch
from scipy import sparse

import faster_weathernext_amd as fwn
from faster_weathernext_amd import hip_attn
from gpu_helpers import MAXTOL, TOL, dev, host
from oracle import attention as A

pytestmark = pytest.mark.gpu
N, D = 256, 128


def _unit_pattern_mask():
  m = np.zeros((N, N), bool)  # m[query, key]
  # Every row has three keys (a band): with a single key, dS is exactly zero and dQ pure rounding.
  for off in (-1, 0, 1):
    m[np.arange(N), (np.arange(N) + off) % N] = True
  # Tile (query block 0, key block 1):
  m[[2, 9, 15], [130, 141, 128]] = True  # keys 128-143 x queries 0-31: half 0 only
  m[[50, 63], [150, 159]] = True  # keys 144-159 x queries 32-63: half 1 only
  m[64:96:4, 160:176:3] = True  # keys 160-191 x queries 64-95: keys 176-191 empty
  m[96:128, 192:208] = True  # a full unit
  m[[100, 120], [210, 220]] = True  # keys 208-223 x queries 96-127: both halves, sparse
  m[127, 255] = True  # a single element
  # Tile (query block 1, key block 0), so that the mask is not symmetric:
  m[200, 5] = True
  m[130:160, 40:48] = True
  return sparse.csr_matrix(m)


def _half_units(dense):
  """Per dK/dV unit (32-query group, 16-key group) of the mask: which 16-query halves are live."""
  h = dense.reshape(N // 32, 2, 16, N // 16, 16).any(axis=(2, 4))  # [query group, half, key group]
  return h[:, 0, :], h[:, 1, :]


@pytest.mark.parametrize("exchange", [True, False])
@pytest.mark.parametrize("precision", ["native", "bf16x3"])
def test_dkv16_unit_patterns(precision, exchange, monkeypatch):
  print(f"dkv16 unit patterns {precision} exchange={exchange}", flush=True)
  mask = _unit_pattern_mask()
  dense = mask.toarray()
  h0, h1 = _half_units(dense)
  assert (h0 & ~h1).any() and (h1 & ~h0).any() and (h0 & h1).any()  # every half case is present
  g32 = dense[64:96, 160:192]
  assert g32[:, :16].any() and not g32[:, 16:].any()  # a 32 x 32 group with one empty 16-key half
  tiles, tiles_t = fwn.TileList.from_mask(mask), fwn.TileList.from_mask(mask.T.tocsr())
  assert tiles.ds_map(tiles_t, hip_attn.unit_keys_for(torch.float32)) is not None  # the exchange can run
  monkeypatch.setattr(hip_attn, "DS_EXCHANGE", exchange)
  rng = np.random.default_rng(11)
  q, k, v, do = (rng.standard_normal((1, N, 2, D)).astype(np.float32) for _ in range(4))
  qt, kt, vt = (dev(x, torch.float32, True) for x in (q, k, v))
  out = fwn.tiled_flash_attention(qt, kt, vt, tiles, scale=D ** -0.5, tiles_t=tiles_t, precision=precision)
  out.backward(dev(do, torch.float32))
  torch.cuda.synchronize()
  got = {"out": host(out), "dq": host(qt.grad), "dk": host(kt.grad), "dv": host(vt.grad)}
  refs = dict(zip(("dq", "dk", "dv"), A.dense_grads(q, k, v, do, dense, D ** -0.5)))
  refs["out"] = A.dense_attention(q, k, v, dense, D ** -0.5)
  # IEEE fp32 products: the float32 bars; bf16x3: rel RMS 1e-5 and max 2e-5 (inputs of standard
  # deviation 1, as in the other bf16x3 tests).
  rms, mx = (TOL[torch.float32], MAXTOL[torch.float32]) if precision == "native" else (1e-5, 2e-5)
  for name, ref in refs.items():
    rr, mr = A.rel_rms(got[name], ref), A.max_rel_err(got[name], ref)
    assert rr <= rms and mr <= mx, (name, rr, mr)
  # Keys with no valid element anywhere get exact zero gradients.
  empty = ~dense.any(axis=0)
  assert not empty.any() or (got["dk"][:, empty] == 0).all()
