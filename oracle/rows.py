"""Row permutation and layer-norm oracle (test infrastructure only).

Restates, in float64 numpy, the steps either side of the reference's layer loop
(``patch.py:274-276, 288-292``):

* ``gather``: ``jnp.take(node_features, perm, axis=1)``.
* ``scatter``: ``jnp.take(x, argsort(perm), axis=1)``, i.e. out[:, perm[i]] = x[:, i].
* ``layer_norm``: ``st.layernorm(x, create_scale=False, create_offset=False)``: (x - mean) /
  sqrt(var + eps) over the last axis with the biased variance. The epsilon of weathernext's
  ``st.layernorm`` is not in the reference tree (weathernext is not vendored); callers pass it.
* ``norm_affine``: layer_norm(x) * mul[:, None] + add[:, None], the per-member affine that
  ``LinearNormConditioning`` applies with its scale and offset.
"""
import numpy as np


def gather(x, perm):
  return np.take(x, perm, axis=1)


def scatter(x, perm):
  out = np.empty_like(x)
  out[:, perm] = x
  return out


def layer_norm(x, eps):
  x = np.asarray(x, np.float64)
  mean = x.mean(-1, keepdims=True)
  var = ((x - mean) ** 2).mean(-1, keepdims=True)
  return (x - mean) / np.sqrt(var + eps)


def norm_affine(x, mul=None, add=None, eps=1e-5):
  y = layer_norm(x, eps)
  if mul is not None:
    y = y * np.asarray(mul, np.float64)[:, None, :]
  if add is not None:
    y = y + np.asarray(add, np.float64)[:, None, :]
  return y
