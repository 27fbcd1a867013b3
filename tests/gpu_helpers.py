"""Shared helpers of the GPU parity tests (inputs as the kernels see them, runs through the op,
and the bars of BASELINE.json)."""
import numpy as np
import torch
from scipy import sparse

import faster_weathernext_amd as fwn
from oracle import attention as A

DEV = "cuda"
# rel RMS bars per output tensor and the reference's unit-test metric
# max|got - ref| / max|ref| (tests/test_pallas_kernel.py:54, 98).
TOL = {torch.float32: 1e-5, torch.bfloat16: 5e-3}
MAXTOL = {torch.float32: 1e-5, torch.bfloat16: 3e-2}


def random_mask(n, density, seed, symmetric=False, identity=True):
  m = sparse.random(n, n, density=density, random_state=seed, format="csr").astype(bool)
  if symmetric:
    m = m + m.T
  if identity:
    m = m + sparse.identity(n, dtype=bool, format="csr")
  return m.tocsr().astype(bool)


def rounded(x, dtype):
  """Inputs as the kernel sees them (bf16 rounding, round to nearest even), back in float32."""
  return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(dtype).float().numpy()


def dev(x, dtype, grad=False):
  t = torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(DEV).to(dtype)
  return t.requires_grad_(grad)


def host(t):
  return t.detach().float().cpu().numpy()


def run(q, k, v, do, tiles, scale, dtype, tiles_t=None):
  """Forward (and backward when do is given) through tiled_flash_attention; float32 numpy results."""
  qt, kt, vt = (dev(x, dtype, do is not None) for x in (q, k, v))
  out = fwn.tiled_flash_attention(qt, kt, vt, tiles, scale=scale, tiles_t=tiles_t)
  res = {"out": host(out)}
  if do is not None:
    out.backward(dev(do, dtype))
    res.update(dq=host(qt.grad), dk=host(kt.grad), dv=host(vt.grad))
  torch.cuda.synchronize()
  return res


def check(got, ref, dtype, what):
  rr, mr = A.rel_rms(got, ref), A.max_rel_err(got, ref)
  assert rr <= TOL[dtype], (what, rr, mr)
  assert mr <= MAXTOL[dtype], (what, rr, mr)


def check_blocks(res, ref, dtype, what=""):
  """Kernel results `res` (full [B, n, H, D] arrays) against block_attention's `ref` at its rows
  (out, dq) and keys (dk, dv)."""
  rows, keys = ref["rows"], ref["keys"]
  if len(rows):
    check(res["out"][:, rows], ref["out"], dtype, (what, "out"))
    if "dq" in res:
      check(res["dq"][:, rows], ref["dq"], dtype, (what, "dq"))
  if len(keys) and "dk" in res:
    check(res["dk"][:, keys], ref["dk"], dtype, (what, "dk"))
    check(res["dv"][:, keys], ref["dv"], dtype, (what, "dv"))
