"""Writes tests/golden/c1_r3_2hop.npz: configuration 1 of the benchmark contract.

Refinement-3 icosahedral mesh (642 nodes), 2-hop mask, batch 1, 2 heads, head_dim 32, float32,
q, k, v, dO ~ N(0, 1) drawn in that order from numpy.random.default_rng(0). Expected outputs are
the float64 dense oracle (oracle/attention.py), stored as float32 (rounding 6e-8, far below the
1e-5 parity bar); lse is stored as float64.

The reference itself cannot run here (jax, haiku and weathernext are not installed), so these
vectors come from the oracle restatement, which tests/test_oracle.py pins independently; the file
also guards the oracle and the mesh construction against drift.

    python tests/golden/make_c1.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import attention as A  # noqa: E402
from oracle import mesh  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c1_r3_2hop.npz")


def make():
  v, f, lat, lon = mesh.icosahedral_mesh(3)
  n = len(v)
  mask = mesh.khop_mask(mesh.adjacency(f, n), 2)
  rng = np.random.default_rng(0)
  q, k, vv, do = (rng.standard_normal((1, n, 2, 32)).astype(np.float32) for _ in range(4))
  scale = 32 ** -0.5
  dense = mask.toarray()
  out = A.dense_attention(q, k, vv, dense, scale)
  lse = A.dense_lse(q, k, dense, scale)
  dq, dk, dv = A.dense_grads(q, k, vv, do, dense, scale)
  np.savez(OUT, indptr=mask.indptr.astype(np.int64), indices=mask.indices.astype(np.int32), q=q, k=k, v=vv,
           do=do, scale=np.float64(scale), out=out.astype(np.float32), lse=lse, dq=dq.astype(np.float32),
           dk=dk.astype(np.float32), dv=dv.astype(np.float32))
  return OUT


if __name__ == "__main__":
  print(make())
