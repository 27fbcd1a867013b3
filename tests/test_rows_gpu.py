"""Parity of the row permutation passes (include/fwn_rows.h) on the GPU.

The gathered copy must be bit-exact. The layer norm is checked against the float64 oracle
(``oracle/rows.py``): float32 within max rel RMS 1e-5, bfloat16 within one bfloat16 rounding of
the float64 value. At the C5 shape ([1, 40962, 768]) the check is the round trip
scatter(gather(x)) against a torch float32 layer norm of x in mesh order.
"""
import numpy as np
import pytest
import torch

from faster_weathernext_amd import rows
from oracle import rows as orows

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _rel_rms(got, ref):
  got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
  return float(np.sqrt(np.mean((got - ref) ** 2)) / max(np.std(ref), 1e-30))


def _bf16_round(a):
  return torch.from_numpy(np.asarray(a, np.float32)).bfloat16().float().numpy()


def _inputs(b, n, c, dtype, seed):
  g = torch.Generator().manual_seed(seed)
  x = (torch.randn(b, n, c, generator=g) * 3 + 1).to(dtype)
  perm = torch.randperm(n, generator=g)
  return x, perm


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("b,n,c", [(1, 1, 8), (2, 7, 64), (1, 300, 768), (3, 33, 1000), (1, 17, 4096), (2, 5, 2056)])
def test_gather_layer_norm_matches_oracle(dtype, b, n, c):
  print(f"gather_layer_norm {dtype} b={b} n={n} c={c}", flush=True)
  x, perm = _inputs(b, n, c, dtype, seed=b * 1000 + n + c)
  xo, no = rows.gather_layer_norm_forward(x.to(DEV), perm.to(DEV), eps=1e-5)
  torch.cuda.synchronize()
  xn = x.float().numpy()
  # the gathered copy is bit-exact
  assert torch.equal(xo.cpu(), x[:, perm])
  ref = orows.layer_norm(orows.gather(xn, perm.numpy()), 1e-5)
  got = no.float().cpu().numpy()
  if dtype == torch.float32:
    assert _rel_rms(got, ref) <= 1e-5
    np.testing.assert_allclose(got, ref, rtol=0, atol=2e-5)
  else:
    # one bfloat16 rounding of a float32 value within 1e-5 of the float64 one
    np.testing.assert_allclose(got, _bf16_round(ref), rtol=2 ** -7, atol=1e-6)
    assert _rel_rms(got, ref) <= 5e-3


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("affine", [False, True])
def test_layer_norm_scatter_matches_oracle(dtype, affine):
  b, n, c = 2, 257, 768
  print(f"layer_norm_scatter {dtype} affine={affine}", flush=True)
  x, perm = _inputs(b, n, c, dtype, seed=7)
  g = torch.Generator().manual_seed(8)
  mul = (1 + 0.1 * torch.randn(b, c, generator=g)) if affine else None
  add = torch.randn(b, c, generator=g) if affine else None
  out = rows.layer_norm_scatter_forward(x.to(DEV), perm.to(DEV), None if mul is None else mul.to(DEV),
                                        None if add is None else add.to(DEV), eps=1e-5)
  torch.cuda.synchronize()
  ref = orows.scatter(orows.norm_affine(x.float().numpy(), None if mul is None else mul.numpy(),
                                        None if add is None else add.numpy(), 1e-5), perm.numpy())
  got = out.float().cpu().numpy()
  if dtype == torch.float32:
    assert _rel_rms(got, ref) <= 1e-5
  else:
    np.testing.assert_allclose(got, _bf16_round(ref), rtol=2 ** -7, atol=1e-5)
    assert _rel_rms(got, ref) <= 5e-3


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("b,n,c", [(1, 1, 8), (2, 257, 768), (3, 33, 1000), (1, 9, 4096)])
def test_layer_norm_affine_matches_oracle(dtype, b, n, c):
  """The block's conditioned layer norm (fwn_rows_norm_affine_launch) against the float64 oracle,
  with and without the affine; rows stay in place."""
  print(f"layer_norm_affine {dtype} b={b} n={n} c={c}", flush=True)
  x, _ = _inputs(b, n, c, dtype, seed=11 + n)
  g = torch.Generator().manual_seed(12)
  mul, add = 1 + 0.1 * torch.randn(b, c, generator=g), torch.randn(b, c, generator=g)
  for m, a in ((mul, add), (None, None), (mul, None)):
    out = rows.layer_norm_affine_forward(x.to(DEV), None if m is None else m.to(DEV), None if a is None else a.to(DEV),
                                         eps=1e-5)
    torch.cuda.synchronize()
    ref = orows.norm_affine(x.float().numpy(), None if m is None else m.numpy(), None if a is None else a.numpy(),
                            1e-5)
    got = out.float().cpu().numpy()
    if dtype == torch.float32:
      assert _rel_rms(got, ref) <= 1e-5
    else:
      np.testing.assert_allclose(got, _bf16_round(ref), rtol=2 ** -7, atol=1e-5)
      assert _rel_rms(got, ref) <= 5e-3


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("b,n,c", [(1, 1, 8), (2, 257, 768), (1, 9, 4096)])
def test_add_layer_norm_affine_matches_separate_ops(dtype, b, n, c):
  """The residual add fused with the conditioned layer norm (fwn_rows_add_norm_affine_launch):
  the sum equals torch's x + y bit for bit (float32 add, one rounding), the normed output equals
  the unfused pass on that sum bit for bit and the float64 oracle to the dtype's bar; also with
  the sum written over x or over y."""
  print(f"add_layer_norm_affine {dtype} b={b} n={n} c={c}", flush=True)
  x, _ = _inputs(b, n, c, dtype, seed=21 + n)
  y, _ = _inputs(b, n, c, dtype, seed=22 + n)
  g = torch.Generator().manual_seed(23)
  mul, add = (1 + 0.1 * torch.randn(b, c, generator=g)).to(DEV), torch.randn(b, c, generator=g).to(DEV)
  xd, yd = x.to(DEV), y.to(DEV)
  want_sum = xd + yd
  want_out = rows.layer_norm_affine_forward(want_sum, mul, add, eps=1e-5)
  with torch.no_grad():
    s, out = rows.add_layer_norm_affine(xd, yd, mul=mul, add=add, eps=1e-5)
    torch.cuda.synchronize()
    assert torch.equal(s, want_sum)
    assert torch.equal(out, want_out)
    ref = orows.norm_affine(want_sum.float().cpu().numpy(), mul.cpu().numpy(), add.cpu().numpy(), 1e-5)
    tol = 1e-5 if dtype == torch.float32 else 5e-3
    assert _rel_rms(out.float().cpu().numpy(), ref) <= tol
    x2 = xd.clone()
    s2, out2 = rows.add_layer_norm_affine(x2, yd, mul=mul, add=add, eps=1e-5, inplace=True)  # sum over x
    torch.cuda.synchronize()
    assert s2.data_ptr() == x2.data_ptr() and torch.equal(x2, want_sum) and torch.equal(out2, want_out)
    y2 = yd.clone()
    L, d = rows.nat.lib(), rows._desc(xd, 1e-5)
    o3 = torch.empty_like(xd)
    rows.nat.check(L.fwn_rows_add_norm_affine_launch(d, xd.data_ptr(), y2.data_ptr(), mul.data_ptr(),
                                                     add.data_ptr(), y2.data_ptr(), o3.data_ptr(),
                                                     rows._stream(xd)))  # sum over y
    torch.cuda.synchronize()
    assert torch.equal(y2, want_sum) and torch.equal(o3, want_out)


def test_add_layer_norm_affine_refuses_autograd():
  x = torch.zeros(1, 4, 8, device=DEV, requires_grad=True)
  with pytest.raises(RuntimeError, match="no derivative"):
    rows.add_layer_norm_affine(x, torch.zeros(1, 4, 8, device=DEV))


def test_layer_norm_affine_gradients_match_torch():
  """Gradients in x, mul and add against the float64 torch composite of the same map."""
  b, n, c = 2, 50, 256
  x, _ = _inputs(b, n, c, torch.float32, seed=13)
  g = torch.Generator().manual_seed(14)
  mul, add = 1 + 0.1 * torch.randn(b, c, generator=g), torch.randn(b, c, generator=g)
  gout = torch.randn(b, n, c, generator=g)
  xs, ms, as_ = (t.to(DEV).requires_grad_(True) for t in (x, mul, add))
  rows.layer_norm_affine(xs, mul=ms, add=as_, eps=1e-5).backward(gout.to(DEV))
  xr, mr, ar = (t.double().requires_grad_(True) for t in (x, mul, add))
  ref = torch.nn.functional.layer_norm(xr, (c,), eps=1e-5) * mr[:, None] + ar[:, None]
  ref.backward(gout.double())
  for got, want in ((xs.grad, xr.grad), (ms.grad, mr.grad), (as_.grad, ar.grad)):
    assert _rel_rms(got.cpu().numpy(), want.numpy()) <= 1e-5


def test_gather_without_norm_and_invalid_entries():
  b, n, c = 2, 40, 64
  x, _ = _inputs(b, n, c, torch.float32, seed=3)
  perm = torch.arange(n).flip(0)
  perm[5] = -1       # out of range: a zero row in the gather, dropped by the scatter
  perm[9] = n + 100
  xd, pd = x.to(DEV), perm.to(DEV)
  xo, no = rows.gather_layer_norm_forward(xd, pd, norm=False)
  assert no is None
  expect = x[:, perm.clamp(0, n - 1)].clone()
  expect[:, [5, 9]] = 0
  assert torch.equal(xo.cpu(), expect)
  # scatter: rows whose target is invalid are dropped; their destinations keep what they held
  out = torch.full_like(xd, 7.0)
  from faster_weathernext_amd import _native as nat
  d = nat.RowsDesc(b, n, c, nat.F32, 1e-5)
  with torch.cuda.device(xd.device):
    nat.check(nat.lib().fwn_rows_norm_scatter_launch(d, xd.data_ptr(), pd.data_ptr(), None, None, out.data_ptr(),
                                                     torch.cuda.current_stream().cuda_stream))
  torch.cuda.synchronize()
  o = out.cpu()
  ln = torch.nn.functional.layer_norm(x, (c,), eps=1e-5)
  for i in range(n):
    if i in (5, 9):
      continue
    torch.testing.assert_close(o[:, perm[i]], ln[:, i], rtol=0, atol=2e-5)
  untouched = [j for j in range(n) if j not in set(perm.tolist())]
  assert untouched and bool((o[:, untouched] == 7.0).all())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_c5_shape_round_trip(dtype):
  """[1, 40962, 768]: the fused gather into Hilbert order and the fused scatter back give the
  layer norm of x in mesh order (size-independent identity), and the gathered copy is exact."""
  from faster_weathernext_amd import mesh
  print(f"c5 round trip {dtype}", flush=True)
  v, f, lat, lon = mesh.icosahedral_mesh(6)
  perm = torch.from_numpy(np.asarray(mesh.hilbert_order(lat, lon), np.int64)).to(DEV)
  n, c = len(lat), 768
  g = torch.Generator(device=DEV).manual_seed(11)
  x = (torch.randn(1, n, c, device=DEV, generator=g) * 2 + 0.5).to(dtype)
  xp, yp = rows.gather_layer_norm_forward(x, perm)
  assert torch.equal(xp, x[:, perm])
  back = rows.layer_norm_scatter_forward(xp, perm)
  ref = torch.nn.functional.layer_norm(x.float(), (c,), eps=1e-5)
  err = (back.float() - ref).square().mean().sqrt() / ref.std()
  assert float(err) <= (1e-5 if dtype == torch.float32 else 5e-3)
  # the gather's norm output is the same layer norm in Hilbert order
  err2 = (yp.float() - ref[:, perm]).square().mean().sqrt() / ref.std()
  assert float(err2) <= (1e-5 if dtype == torch.float32 else 5e-3)


def test_gradients_match_torch_composite():
  b, n, c = 2, 96, 128
  print("row pass gradients", flush=True)
  g = torch.Generator().manual_seed(5)
  x0 = torch.randn(b, n, c, generator=g, dtype=torch.float64)
  perm = torch.randperm(n, generator=g)
  mul0 = 1 + 0.2 * torch.randn(b, c, generator=g, dtype=torch.float64)
  add0 = torch.randn(b, c, generator=g, dtype=torch.float64)
  gx = torch.randn(b, n, c, generator=g, dtype=torch.float64)
  gn = torch.randn(b, n, c, generator=g, dtype=torch.float64)
  go = torch.randn(b, n, c, generator=g, dtype=torch.float64)

  # float64 reference (CPU): composite of index_select and layer_norm
  x = x0.clone().requires_grad_(True)
  mul, add = mul0.clone().requires_grad_(True), add0.clone().requires_grad_(True)
  xp = x[:, perm]
  yp = torch.nn.functional.layer_norm(xp, (c,), eps=1e-5)
  z = torch.nn.functional.layer_norm(x, (c,), eps=1e-5) * mul[:, None] + add[:, None]
  inv = torch.argsort(perm)
  out = z[:, inv]
  ((xp * gx).sum() + (yp * gn).sum() + (out * go).sum()).backward()
  ref_x, ref_mul, ref_add = x.grad, mul.grad, add.grad

  xd = x0.float().to(DEV).requires_grad_(True)
  muld = mul0.float().to(DEV).requires_grad_(True)
  addd = add0.float().to(DEV).requires_grad_(True)
  pd = perm.to(DEV)
  xo, no = rows.gather_layer_norm(xd, pd)
  od = rows.layer_norm_scatter(xd, pd, mul=muld, add=addd)
  ((xo * gx.float().to(DEV)).sum() + (no * gn.float().to(DEV)).sum() + (od * go.float().to(DEV)).sum()).backward()
  for got, ref in ((xd.grad, ref_x), (muld.grad, ref_mul), (addd.grad, ref_add)):
    assert _rel_rms(got.double().cpu().numpy(), ref.numpy()) <= 1e-5
