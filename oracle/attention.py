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
* ``block_attention`` / ``sampled_attention``: the dense closed form evaluated only at whole
  128-row / 128-key blocks, or at single rows and keys, of masks too large for ``dense_*``
  (refinement-6 meshes); pinned against ``dense_*`` on small masks.
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

  qc [B, H, chunk, D] and kc [B, H, window, D] are head-major. The softmax runs in at least
  float32, as the reference's upcast wrapper does (``patch.py:151``); float64 stays float64.
  """
  logits = np.matmul(qc, kc.transpose(0, 1, 3, 2)) * qc.dtype.type(scale)
  valid = np.unpackbits(packed, axis=-1, count=window, bitorder="little").astype(bool)
  soft = np.promote_types(logits.dtype, np.float32)
  logits = np.where(valid[None, None], logits, logits.dtype.type(MASK_VALUE)).astype(soft, copy=False)
  logits -= logits.max(-1, keepdims=True)
  np.exp(logits, out=logits)
  logits /= logits.sum(-1, keepdims=True)
  return logits.astype(qc.dtype, copy=False)


def _head_major(x):
  return np.ascontiguousarray(x.transpose(0, 2, 1, 3))


def chunked_attention(q, k, v, starts, bits, window, n_kv, chunk, scale, chunks=None):
  """Reference XLA chunked path, forward: [B, n, H, D] in q's dtype.

  ``chunks`` (optional iterable of chunk indices) restricts the work to those query chunks; rows
  of other chunks are left at zero (used for bounded CPU-baseline samples).
  """
  n = q.shape[1]
  qp, kp, vp = (_head_major(x) for x in _chunk_views(q, k, v, starts, window, n_kv, chunk))
  out = np.zeros_like(qp)
  for c in (range(len(starts)) if chunks is None else chunks):
    s0 = int(starts[c])
    rows = slice(c * chunk, (c + 1) * chunk)
    w = _chunk_probs(qp[:, :, rows], kp[:, :, s0:s0 + window], bits[c], window, scale)
    out[:, :, rows] = np.matmul(w, vp[:, :, s0:s0 + window])
  return out.transpose(0, 2, 1, 3)[:, :n]


def chunked_attention_grads(q, k, v, do, starts, bits, window, n_kv, chunk, scale, chunks=None):
  """Reference XLA chunked path, backward (autodiff of the chunked forward): (dq, dk, dv)."""
  n = q.shape[1]
  qp, kp, vp = (_head_major(x) for x in _chunk_views(q, k, v, starts, window, n_kv, chunk))
  dop = np.zeros(qp.shape, do.dtype)
  dop[:, :, :n] = do.transpose(0, 2, 1, 3)
  dq, dk, dv = np.zeros_like(qp), np.zeros_like(kp), np.zeros_like(vp)
  sc = q.dtype.type(scale)
  for c in (range(len(starts)) if chunks is None else chunks):
    s0 = int(starts[c])
    rows, keys = slice(c * chunk, (c + 1) * chunk), slice(s0, s0 + window)
    qc, doc, kc, vc = qp[:, :, rows], dop[:, :, rows], kp[:, :, keys], vp[:, :, keys]
    p = _chunk_probs(qc, kc, bits[c], window, scale)
    dp = np.matmul(doc, vc.transpose(0, 1, 3, 2))
    dp -= (dp * p).sum(-1, keepdims=True)
    dp *= p                                                     # dS
    dq[:, :, rows] = np.matmul(dp, kc) * sc
    dk[:, :, keys] += np.matmul(dp.transpose(0, 1, 3, 2), qc) * sc
    dv[:, :, keys] += np.matmul(p.transpose(0, 1, 3, 2), doc)
  return tuple(x.transpose(0, 2, 1, 3)[:, :n] for x in (dq, dk, dv))


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


def block_attention(q, k, v, do, mask, scale, row_blocks=(), key_blocks=(), block=128):
  """Exact float64 results for whole blocks of 128 rows and of 128 keys of a large sparse mask.

  The closed form of ``dense_attention`` / ``dense_grads``, evaluated one query block at a time
  over the distinct keys that block's rows attend to (the 128-row unit of the kernels' tile list,
  ``pallas_attn.py:85-109``): for query block b, S = Q_b K_C^T scale over its key set C, the masked
  softmax P, O = P V_C and lse; delta_i = dO_i . O_i (= rowsum(P o dP)); dP = dO V^T, dS =
  P (dP - delta). ``row_blocks`` receive out, lse and dq of all their rows. ``key_blocks`` receive
  dk = scale dS^T Q and dv = P^T dO summed over every query block with a row that attends to one
  of their keys (each query block is evaluated once for all requested key blocks). Rows with no
  valid key get zero output and gradients (the kernels' convention).

  Returns a dict: out/dq [B, rows, H, D] and lse [B, H, rows] over the concatenated rows of
  ``row_blocks`` (ragged last block included as far as n), dk/dv [B, keys, H, D] over the
  concatenated keys of ``key_blocks``; ``rows`` and ``keys`` hold the node indices.
  """
  mask = sparse.csr_matrix(mask).astype(bool)
  n = mask.shape[0]
  hm = lambda x: np.ascontiguousarray(np.asarray(x, np.float64).transpose(0, 2, 1, 3))  # [B, H, n, D]
  qh, kh, vh, doh = hm(q), hm(k), hm(v), hm(do)
  span = lambda b: np.arange(b * block, min(n, (b + 1) * block))
  rows = np.concatenate([span(b) for b in row_blocks]) if len(row_blocks) else np.zeros(0, np.int64)
  keys = np.concatenate([span(b) for b in key_blocks]) if len(key_blocks) else np.zeros(0, np.int64)
  B, H, _, D = qh.shape
  out = np.zeros((B, H, len(rows), D))
  dq = np.zeros_like(out)
  lse = np.zeros((B, H, len(rows)))
  dk = np.zeros((B, H, len(keys), D))
  dv = np.zeros_like(dk)
  # Query blocks holding a row that attends to one of the requested keys.
  need = set(int(b) for b in row_blocks)
  for kb in key_blocks:
    hit = mask[:, kb * block:min(n, (kb + 1) * block)].tocoo().row
    need.update(int(b) for b in np.unique(hit // block))
  row_pos = {int(b): i for i, b in enumerate(row_blocks)}
  key_pos = np.full(n, -1, np.int64)
  key_pos[keys] = np.arange(len(keys))
  row_off = np.concatenate([[0], np.cumsum([len(span(b)) for b in row_blocks])]).astype(int)
  for qb in sorted(need):
    r = span(qb)
    sub = mask[r[0]:r[-1] + 1]
    cols = np.unique(sub.indices)
    if len(cols) == 0:
      continue
    valid = sub[:, cols].toarray()                                           # [rows, C]
    p = np.matmul(qh[:, :, r], kh[:, :, cols].transpose(0, 1, 3, 2))         # [B, H, rows, C]
    p *= scale
    np.copyto(p, -np.inf, where=~valid)
    mx = p.max(-1, keepdims=True)
    has = np.isfinite(mx)
    mx[~has] = 0.0
    p -= mx
    np.exp(p, out=p)
    tot = p.sum(-1, keepdims=True)
    tot[~has] = 1.0
    p /= tot
    o = np.matmul(p, vh[:, :, cols])                                         # [B, H, rows, D]
    delta = (o * doh[:, :, r]).sum(-1, keepdims=True)
    if qb in row_pos:
      a, b_ = row_off[row_pos[qb]], row_off[row_pos[qb] + 1]
      dp = np.matmul(doh[:, :, r], vh[:, :, cols].transpose(0, 1, 3, 2))
      out[:, :, a:b_] = o
      dq[:, :, a:b_] = np.matmul(p * (dp - delta), kh[:, :, cols]) * scale
      lse[:, :, a:b_] = np.where(has, mx + np.log(tot), -np.inf)[..., 0]
    # Contributions of this query block to the requested keys it attends to.
    sel = np.flatnonzero(key_pos[cols] >= 0)
    if len(sel) == 0:
      continue
    kpos = key_pos[cols[sel]]
    psel = p[..., sel]                                                       # [B, H, rows, S]
    dpsel = np.matmul(doh[:, :, r], vh[:, :, cols[sel]].transpose(0, 1, 3, 2))
    dssel = psel * (dpsel - delta)
    dk[:, :, kpos] += np.matmul(dssel.transpose(0, 1, 3, 2), qh[:, :, r]) * scale
    dv[:, :, kpos] += np.matmul(psel.transpose(0, 1, 3, 2), doh[:, :, r])
  nm = lambda x: x.transpose(0, 2, 1, 3)
  return {"out": nm(out), "dq": nm(dq), "lse": lse, "dk": nm(dk), "dv": nm(dv), "rows": rows, "keys": keys}


def sampled_attention(q, k, v, do, mask, scale, rows, keys=()):
  """Exact float64 results at a sample of rows and keys, for masks too large for the dense oracle.

  Same closed form as ``dense_attention`` / ``dense_grads``, evaluated only where needed: out, lse
  and dq at query ``rows`` (each needs its own key set), dk and dv at ``keys`` (each needs every
  query that attends to it, and those queries' normalisers). Returns a dict of arrays
  out/dq [B, len(rows), H, D], lse [B, H, len(rows)], dk/dv [B, len(keys), H, D].
  """
  mask = sparse.csr_matrix(mask).astype(bool)
  mask_t = mask.T.tocsr()
  q, k, v, do = (np.asarray(x, np.float64) for x in (q, k, v, do))
  cache = {}

  def row(i):
    if i not in cache:
      cols = mask.indices[mask.indptr[i]:mask.indptr[i + 1]]
      s = np.einsum("bhd,bmhd->bhm", q[:, i], k[:, cols]) * scale
      mx = s.max(-1, keepdims=True)
      e = np.exp(s - mx)
      tot = e.sum(-1, keepdims=True)
      p = e / tot
      dp = np.einsum("bhd,bmhd->bhm", do[:, i], v[:, cols])
      ds = p * (dp - (p * dp).sum(-1, keepdims=True))
      cache[i] = dict(cols=cols, p=p, ds=ds, lse=(mx + np.log(tot))[..., 0])
    return cache[i]

  res = {"out": [], "lse": [], "dq": [], "dk": [], "dv": []}
  for i in rows:
    r = row(int(i))
    res["out"].append(np.einsum("bhm,bmhd->bhd", r["p"], v[:, r["cols"]]))
    res["dq"].append(np.einsum("bhm,bmhd->bhd", r["ds"], k[:, r["cols"]]) * scale)
    res["lse"].append(r["lse"])
  for j in keys:
    j = int(j)
    dk = np.zeros(q.shape[:1] + q.shape[2:])
    dv = np.zeros_like(dk)
    for i in mask_t.indices[mask_t.indptr[j]:mask_t.indptr[j + 1]]:
      r = row(int(i))
      pos = np.searchsorted(r["cols"], j)
      dv += r["p"][..., pos, None] * do[:, i]
      dk += r["ds"][..., pos, None] * q[:, i] * scale
    res["dk"].append(dk)
    res["dv"].append(dv)
  out = {}
  for name in ("out", "dq", "dk", "dv"):
    out[name] = np.stack(res[name], 1) if res[name] else np.zeros(q.shape[:1] + (0,) + q.shape[2:])
  out["lse"] = np.stack(res["lse"], -1) if res["lse"] else np.zeros(q.shape[:1] + q.shape[2:3] + (0,))
  return out
