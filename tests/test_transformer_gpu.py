"""The mesh transformer wiring (``transformer.MeshTransformer``) against the same model written
with plain torch operations: a dense masked softmax in place of the HIP attention, and separate
gather / layer-norm / scatter steps in place of the fused row passes (``patch.py:233-292``).
Same weights; float32; the check is max rel RMS over the output, the input gradient and every
parameter gradient."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import faster_weathernext_amd as fwn

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _reference(model, mask, x, cond):
  d = x.shape[-1]
  perm = model.perm
  xp = x[:, perm] if perm is not None else x
  allowed = torch.from_numpy(mask).to(x.device)
  for blk in model.blocks:
    h = blk.norm_mha(F.layer_norm(xp, (d,), eps=model.eps), cond)
    b, n, _ = h.shape
    H, Dk = blk.mha.num_heads, blk.mha.key_size
    q, k, v = blk.mha.qkv(h).view(b, n, 3, H, Dk).unbind(2)
    s = torch.einsum("bnhd,bmhd->bhnm", q, k) * Dk ** -0.5
    p = torch.softmax(s.masked_fill(~allowed, float("-inf")), dim=-1)
    o = torch.einsum("bhnm,bmhd->bnhd", p, v).reshape(b, n, H * Dk)
    xp = xp + blk.mha.final(o)
    xp = xp + blk.ffw(blk.norm_ffw(F.layer_norm(xp, (d,), eps=model.eps), cond))
  mul, add = model.final_norm.affine(cond)
  y = F.layer_norm(xp, (d,), eps=model.eps) * mul[:, None] + add[:, None]
  if perm is None:
    return y
  out = torch.empty_like(y)
  out[:, perm] = y
  return out


def _rel_rms(a, b):
  return float((a - b).square().mean().sqrt() / b.std())


def _directed_adjacency(refinement, seed):
  """The mesh adjacency with 30% of its directed edges dropped: not symmetric."""
  from scipy import sparse
  v, f, lat, lon = fwn.icosahedral_mesh(refinement)
  coo = fwn.adjacency(f, len(v)).tocoo()
  keep = np.random.default_rng(seed).random(coo.nnz) < 0.7
  adj = sparse.csr_matrix((np.ones(int(keep.sum()), bool), (coo.row[keep], coo.col[keep])), shape=(len(v), len(v)))
  return adj, lat, lon


@pytest.mark.parametrize("case", ["hilbert", "subdivision", "directed", "bf16x3"])
def test_mesh_transformer_matches_plain_torch(case):
  """"directed" builds the model from a non-symmetric adjacency: its mask is not symmetric, so the
  backward walks the transposed tile list the model builds (patch.py:215-218). "bf16x3" is the
  Hilbert case with the attention's products in the split precision (bar 3e-5: each operand
  carries about 16 significant bits, over three layers)."""
  print(f"mesh transformer {case}", flush=True)
  reorder = case != "subdivision"
  tol = 3e-5 if case == "bf16x3" else 1e-5
  torch.manual_seed(0)
  kw = dict(refinement=3, k_hop=2, num_layers=3, d_model=64, num_heads=2, key_size=32, ffw_hidden=128, cond_size=8,
            reorder=reorder, device=DEV, dtype=torch.float32,
            precision="bf16x3" if case == "bf16x3" else "native")
  if case == "directed":
    adj, lat, lon = _directed_adjacency(3, 1)
    model = fwn.MeshTransformer(adjacency=adj, latlon=(lat, lon), **kw)
    assert model.tiles_t is not None
  else:
    model = fwn.MeshTransformer(**kw)
  with torch.no_grad():  # the conditioning starts at zero; give it weights so it is exercised
    for mod in model.modules():
      if isinstance(mod, fwn.transformer.NormConditioning):
        mod.linear.weight.normal_(0, 0.1)
        mod.linear.bias.normal_(0, 0.1)
  if case == "directed":
    mask, perm = fwn.khop_mask(adj, 2), fwn.hilbert_order(lat, lon)
  else:
    mask, lat, lon, perm = fwn.mesh_mask(3, 2, reorder=reorder)
  dense = (mask[perm][:, perm] if perm is not None else mask).toarray()
  assert (case == "directed") == bool((dense != dense.T).any())
  n = mask.shape[0]
  x = torch.randn(2, n, 64, device=DEV, requires_grad=True)
  cond = torch.randn(2, 8, device=DEV)
  g = torch.randn(2, n, 64, device=DEV)
  out = model(x, cond)
  out.backward(g)
  gx = x.grad.clone()
  grads = {name: p.grad.clone() for name, p in model.named_parameters()}
  x.grad = None
  model.zero_grad(set_to_none=True)
  ref = _reference(model, dense, x, cond)
  ref.backward(g)
  assert _rel_rms(out.detach(), ref.detach()) <= tol
  assert _rel_rms(gx, x.grad) <= tol
  with torch.no_grad():  # inference path: GELU in the feed-forward GEMM's epilogue
    assert _rel_rms(model(x, cond), ref.detach()) <= tol
  # every parameter, the conditioning projections included (their gradients flow through the
  # fused conditioned layer norms)
  for name, p in model.named_parameters():
    assert _rel_rms(grads[name], p.grad) <= tol, name
