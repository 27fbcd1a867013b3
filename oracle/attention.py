"""Masked softmax attention oracles (test infrastructure only).

Layouts follow the reference's public op: q, k, v, dO are [B, n, H, D] (node-major), the mask is
a boolean [n, n] (query row, key column) shared by every batch element and head
(``pallas_attn.py:317-328``).

* ``dense_attention`` / ``dense_grads``: float64 closed form, masked logits = -inf
  (``tests/test_pallas_kernel.py:15-21, 58-69``). ``dense_lse`` is the per-row log-sum-exp the
  forward kernel saves for the backward (``pallas_attn.py:140-141``).
* ``build_chunked_mask`` / ``chunked_attention`` / ``chunked_attention_grads``: the reference XLA
  chunked banded-window path (``patch.py:106-162``; the same maths in
  ``scripts/attn_bench.py:55-77``): queries in chunks of ``chunk``, each against one contiguous
  key window, masked logits = -1e30, softmax in float32, then times V. The backward is what
  autodiff of that path computes (chunks rematerialised, ``scripts/attn_bench.py:76``):
  dS = P * (dP - rowsum(dP * P)), dQ = dS K s, dK += dS^T Q s, dV += P^T dO per window.
  These run in the input's float dtype (float32 for the CPU baseline).
"""

import numpy as np
from scipy import sparse

MASK_VALUE = -1e30


def _dense_probs(q, k, mask, scale):
  """P [B, H, n, n] float64 of masked softmax."""
  s = np.einsum("bnhd,bmhd->bhnm", q.astype(np.float64), k.astype(np.float64)) * scale
  s = np.where(mask[None, None], s, -np.inf)
  m = s.max(-1, keepdims=True)
  p = np.exp(s - m)
  return p / p.sum(-1, keepdims=True)


def dense_attention(q, k, v, mask, scale):
  """float64 [B, n, H, D] output of softmax(mask(q k^T * scale)) v."""
  p = _dense_probs(q, k, mask, scale)
  return np.einsum("bhnm,bmhd->bnhd", p, v.astype(np.float64))


def dense_lse(q, k, mask, scale):
  """float64 [B, H, n] log-sum-exp of the masked, scaled logits of each query row."""
  s = np.einsum("bnhd,bmhd->bhnm", q.astype(np.float64), k.astype(np.float64)) * scale
  s = np.where(mask[None, None], s, -np.inf)
  m = s.max(-1, keepdims=True)
  return (m + np.log(np.exp(s - m).sum(-1, keepdims=True)))[..., 0]


def dense_grads(q, k, v, do, mask, scale):
  """float64 (dq, dk, dv), each [B, n, H, D], of sum(out * do) for the masked softmax attention."""
  p = _dense_probs(q, k, mask, scale)
  q, k, v, do = (x.astype(np.float64) for x in (q, k, v, do))
  dp = np.einsum("bnhd,bmhd->bhnm", do, v)
  ds = p * (dp - (dp * p).sum(-1, keepdims=True))
  dq = np.einsum("bhnm,bmhd->bnhd", ds, k) * scale
  dk = np.einsum("bhnm,bnhd->bmhd", ds, q) * scale
  dv = np.einsum("bhnm,bnhd->bmhd", p, do)
  return dq, dk, dv


def build_chunked_mask(mask, chunk):
  """(starts int32[n_chunks], bits uint8[n_chunks, chunk, window // 8], window, n_kv).

  Restates ``patch.py:106-127``: one contiguous key window per chunk of queries, the window the
  widest chunk span rounded up to 128, start clipped so the window stays inside n_kv; the mask
  of each chunk is packed little-endian along the window.
  """
  mask = sparse.csr_matrix(mask).astype(bool)
  n = mask.shape[0]
  n_chunks = -(-n // chunk)
  lo = np.array([mask.indices[mask.indptr[i]:mask.indptr[i + 1]].min() for i in range(n)])
  hi = np.array([mask.indices[mask.indptr[i]:mask.indptr[i + 1]].max() for i in range(n)])
  span = max(hi[c * chunk:(c + 1) * chunk].max() - lo[c * chunk:(c + 1) * chunk].min() + 1
             for c in range(n_chunks))
  window = int(-(-span // 128) * 128)
  n_kv = max(n, window)
  wide = sparse.hstack([mask, sparse.csr_matrix((n, n_kv - n), dtype=bool)]).tocsr()
  starts = np.zeros(n_chunks, np.int32)
  bits = np.zeros((n_chunks, chunk, window // 8), np.uint8)
  for c in range(n_chunks):
    r0, r1 = c * chunk, min((c + 1) * chunk, n)
    starts[c] = min(lo[r0:r1].min(), n_kv - window)
    block = wide[r0:r1, starts[c]:starts[c] + window].toarray()
    assert block.sum() == wide[r0:r1].sum(), f"chunk {c} window too narrow"
    bits[c, :r1 - r0] = np.packbits(block, axis=-1, bitorder="little")
  return starts, bits, window, n_kv


def _chunk_views(q, k, v, starts, window, n_kv, chunk):
  batch, n, heads, dim = q.shape
  n_chunks = len(starts)
  qp = np.zeros((batch, n_chunks * chunk, heads, dim), q.dtype)
  qp[:, :n] = q
  kp = np.zeros((batch, n_kv, heads, dim), k.dtype)
  vp = np.zeros((batch, n_kv, heads, dim), v.dtype)
  kp[:, :n], vp[:, :n] = k, v
  return qp, kp, vp


def _chunk_probs(qc, kc, packed, window, scale):
  """Softmax weights [B, H, chunk, window] of one chunk, masked logits = -1e30.

  The softmax runs in at least float32, as the reference's upcast wrapper does
  (``patch.py:151``); float64 inputs stay float64.
  """
  logits = np.einsum("bqhd,bkhd->bhqk", qc, kc) * qc.dtype.type(scale)
  valid = np.unpackbits(packed, axis=-1, count=window, bitorder="little").astype(bool)
  soft = np.promote_types(logits.dtype, np.float32)
  logits = np.where(valid[None, None], logits, logits.dtype.type(MASK_VALUE)).astype(soft)
  m = logits.max(-1, keepdims=True)
  p = np.exp(logits - m)
  return (p / p.sum(-1, keepdims=True)).astype(qc.dtype), valid


def chunked_attention(q, k, v, starts, bits, window, n_kv, chunk, scale, chunks=None):
  """Reference XLA chunked path, forward: [B, n, H, D] in q's dtype.

  ``chunks`` (optional iterable of chunk indices) restricts the work to those query chunks; rows
  of other chunks are left at zero (used for bounded CPU-baseline samples).
  """
  batch, n, heads, dim = q.shape
  qp, kp, vp = _chunk_views(q, k, v, starts, window, n_kv, chunk)
  out = np.zeros_like(qp)
  for c in (range(len(starts)) if chunks is None else chunks):
    s0 = int(starts[c])
    qc = qp[:, c * chunk:(c + 1) * chunk]
    kc, vc = kp[:, s0:s0 + window], vp[:, s0:s0 + window]
    w, _ = _chunk_probs(qc, kc, bits[c], window, scale)
    out[:, c * chunk:(c + 1) * chunk] = np.einsum("bhqk,bkhd->bqhd", w, vc)
  return out[:, :n]


def chunked_attention_grads(q, k, v, do, starts, bits, window, n_kv, chunk, scale, chunks=None):
  """Reference XLA chunked path, backward (autodiff of the chunked forward): (dq, dk, dv)."""
  batch, n, heads, dim = q.shape
  qp, kp, vp = _chunk_views(q, k, v, starts, window, n_kv, chunk)
  dop = np.zeros_like(qp)
  dop[:, :n] = do
  dq = np.zeros_like(qp)
  dk = np.zeros_like(kp)
  dv = np.zeros_like(vp)
  sc = q.dtype.type(scale)
  for c in (range(len(starts)) if chunks is None else chunks):
    s0 = int(starts[c])
    rows = slice(c * chunk, (c + 1) * chunk)
    qc, doc = qp[:, rows], dop[:, rows]
    kc, vc = kp[:, s0:s0 + window], vp[:, s0:s0 + window]
    p, _ = _chunk_probs(qc, kc, bits[c], window, scale)
    dp = np.einsum("bqhd,bkhd->bhqk", doc, vc)
    ds = p * (dp - (dp * p).sum(-1, keepdims=True))
    dq[:, rows] = np.einsum("bhqk,bkhd->bqhd", ds, kc) * sc
    dk[:, s0:s0 + window] += np.einsum("bhqk,bqhd->bkhd", ds, qc) * sc
    dv[:, s0:s0 + window] += np.einsum("bhqk,bqhd->bkhd", p, doc)
  return dq[:, :n], dk[:, :n], dv[:, :n]


def rel_rms(got, ref):
  """RMS(got - ref) / std(ref), the reference's comparison metric (``scripts/attn_bench.py:122``)."""
  got = np.asarray(got, np.float64)
  ref = np.asarray(ref, np.float64)
  return float(np.sqrt(np.mean((got - ref) ** 2)) / ref.std())


def max_rel_err(got, ref):
  """max|got - ref| / max|ref|, the reference's unit-test metric (``tests/test_pallas_kernel.py:54``)."""
  got = np.asarray(got, np.float64)
  ref = np.asarray(ref, np.float64)
  return float(np.abs(got - ref).max() / np.abs(ref).max())
