"""CPU oracle for block-sparse masked mesh attention (test infrastructure only).

This package restates, on the CPU and in float64 where it matters, what the reference
(Raymondlol/Faster-WeatherNext v0.2.0) computes on the hot path:

* ``mesh``      icosahedral mesh, adjacency and k-hop neighbourhood mask
                (``scripts/attn_bench.py:26-33``; ``patch.py:209``).
* ``tiles``     Hilbert ordering and the CSR live-tile list (``pallas_attn.py:41-109``).
* ``attention`` dense masked softmax attention and its analytic gradients
                (``tests/test_pallas_kernel.py:15-21, 58-69``), and the reference XLA chunked path
                (``patch.py:106-162``, ``scripts/attn_bench.py:55-77``) with its backward.
* ``rows``      the Hilbert gather/scatter of the node features either side of the layer loop
                and the layer norms next to them (``patch.py:244, 274-276, 288-292``).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import this package, and only as the checker or the timed CPU baseline. The product
(``faster-weathernext_amd/``) never imports it and has no CPU fallback.

How each function is pinned (checks live in ``tests/test_oracle.py``):

* ``attention.dense_attention`` / ``dense_grads``: closed form; brute-force per-row softmax on tiny
  inputs; rows of P sum to 1; masked keys get zero weight and zero dK/dV; a float64 finite
  difference of a scalar loss; dV = P^T dO and dQ linear in dO.
* ``attention.chunked_attention`` / ``chunked_attention_grads`` / ``build_chunked_mask``: equal to
  the dense oracle on the same inputs; chunked-mask round trip (``tests/test_masks.py:55-66``).
* ``mesh.icosahedral_mesh`` / ``khop_mask``: V = 10*4^r + 2, E = 30*4^r, F = 20*4^r; Euler
  characteristic 2; 12 vertices of degree 5, the rest degree 6; unit-norm vertices; symmetric
  mask; BFS ball sizes against the hexagonal closed form 1 + 3k(k+1) away from pentagons; the
  reference's logged mean of 3,101 keys per query for the 32-hop mask at refinement 6
  (``docs/results/attn_bwd/attn_bwd_default_rtx5090.txt:3``).
* ``tiles.hilbert_order``: the Hilbert-curve properties on a brute-forced 2^b cube (bijection,
  unit steps between consecutive cells, origin first) and the invariants of
  ``tests/test_masks.py:39-52``.
* ``tiles.build_tile_mask``: dense round trip and distinct non-empty tiles per block
  (``tests/test_masks.py:25-36``).
* ``rows.gather`` / ``scatter``: scatter inverts gather for the same permutation, and gather
  with the identity is the identity. ``rows.layer_norm``: every row has mean 0 and variance
  var / (var + eps); it is invariant to adding a constant to a row and to scaling it by a
  positive factor when eps = 0; on a two-value row it reduces to +-1 in closed form.
"""
