"""GPU tests of the C ABI itself (include/fwn_attn.h), called through ctypes as a JAX-free harness
or an XLA FFI handler would call it: the one-stream backward fwn_attn_bwd_launch, and capture of
the launchers into a graph that is replayed.
"""
import ctypes

import numpy as np
import pytest
import torch

import faster_weathernext_amd as fwn
from faster_weathernext_amd import _native as nat
from gpu_helpers import check, dev, host, random_mask, rounded
from oracle import attention as A

pytestmark = pytest.mark.gpu
DT = {torch.float32: nat.F32, torch.bfloat16: nat.BF16}


def _ws_size(desc, *lists):
  size = 0
  for tl in lists:
    n = ctypes.c_uint64(0)
    nat.check(nat.lib().fwn_attn_workspace_size(desc, tl.struct, ctypes.byref(n)))
    size = max(size, int(n.value))
  return size


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("split", [False, True])
def test_bwd_launch_one_stream(split, dtype, monkeypatch):
  """fwn_attn_bwd_launch (delta, dq, then dk/dv on one stream, one workspace sized for the larger
  of the two lists) on a non-symmetric mask with its transposed list. Split schedules cut every
  block into items of at most 2 (forward list) and 3 (transposed list) tiles. The results equal
  the package's recomputing backward (the same kernels on two streams, each with its own
  workspace) bit for bit and the dense float64 oracle within the bars."""
  monkeypatch.setattr(fwn.hip_attn, "DS_EXCHANGE", False)
  rng = np.random.default_rng(60)
  b, n, h, d = 2, 700, 2, 64
  q, k, v, do = (rounded(rng.standard_normal((b, n, h, d)), dtype) for _ in range(4))
  m = random_mask(n, 0.05, 61, symmetric=False)
  cap, cap_t = (2, 3) if split else (1 << 20, 1 << 20)
  tiles = fwn.TileList.from_mask(m, max_item_tiles=cap)
  tiles_t = fwn.TileList.from_mask(m.T.tocsr(), max_item_tiles=cap_t)
  assert (tiles.n_split > 0 and tiles_t.n_split > 0) == split
  qd, kd, vd, dod = (dev(x, dtype) for x in (q, k, v, do))
  scale = d ** -0.5
  out, lse = fwn.attention_forward(qd, kd, vd, tiles, scale)
  desc = nat.AttnDesc(b, n, h, d, DT[dtype], scale, *qd.stride()[:3])
  size = _ws_size(desc, tiles, tiles_t)
  assert (size > 0) == split
  ws = torch.full((max(size, 1),), 255, dtype=torch.uint8, device="cuda")
  delta = torch.full((b, h, n), float("nan"), device="cuda")
  dq, dk, dv = (torch.full_like(qd, float("nan")) for _ in range(3))
  stream = torch.cuda.current_stream().cuda_stream
  nat.check(nat.lib().fwn_attn_bwd_launch(desc, qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), out.data_ptr(),
                                          dod.data_ptr(), lse.data_ptr(), delta.data_ptr(), tiles.struct,
                                          tiles_t.struct, dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                                          ws.data_ptr() if size else None, size, stream))
  ref = fwn.attention_backward(qd, kd, vd, out, lse, dod, tiles, tiles_t, scale)
  torch.cuda.synchronize()
  for name, got, want in zip(("dq", "dk", "dv"), (dq, dk, dv), ref):
    np.testing.assert_array_equal(host(got), host(want), err_msg=name)
  np.testing.assert_allclose(host(delta), (host(out) * do).sum(-1).transpose(0, 2, 1), rtol=1e-5, atol=1e-4)
  dense = A.dense_grads(q, k, v, do, m.toarray(), scale)
  for name, got, want in zip(("dq", "dk", "dv"), (dq, dk, dv), dense):
    check(host(got), want, dtype, name)


def test_bwd_launch_without_transposed_list_uses_the_forward_list(monkeypatch):
  """tiles_t = NULL means the forward list (a symmetric mask), as the reference's tiles_t=None."""
  monkeypatch.setattr(fwn.hip_attn, "DS_EXCHANGE", False)
  rng = np.random.default_rng(62)
  b, n, h, d = 1, 400, 2, 32
  q, k, v, do = (rounded(rng.standard_normal((b, n, h, d)), torch.bfloat16) for _ in range(4))
  m = random_mask(n, 0.05, 63, symmetric=True)
  tiles = fwn.TileList.from_mask(m, max_item_tiles=2)
  qd, kd, vd, dod = (dev(x, torch.bfloat16) for x in (q, k, v, do))
  out, lse = fwn.attention_forward(qd, kd, vd, tiles, d ** -0.5)
  desc = nat.AttnDesc(b, n, h, d, nat.BF16, d ** -0.5, *qd.stride()[:3])
  size = _ws_size(desc, tiles)
  ws = torch.empty(size, dtype=torch.uint8, device="cuda")
  delta = torch.empty((b, h, n), device="cuda")
  dq, dk, dv = (torch.empty_like(qd) for _ in range(3))
  nat.check(nat.lib().fwn_attn_bwd_launch(desc, qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), out.data_ptr(),
                                          dod.data_ptr(), lse.data_ptr(), delta.data_ptr(), tiles.struct, None,
                                          dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), ws.data_ptr(), size,
                                          torch.cuda.current_stream().cuda_stream))
  ref = fwn.attention_backward(qd, kd, vd, out, lse, dod, tiles, None, d ** -0.5)
  torch.cuda.synchronize()
  for name, got, want in zip(("dq", "dk", "dv"), (dq, dk, dv), ref):
    np.testing.assert_array_equal(host(got), host(want), err_msg=name)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("split", [False, True])
def test_bwd_ds_launch_one_stream(split, dtype):
  """fwn_attn_bwd_ds_launch (delta, dk/dv writing dS, then dq from dS, on one stream) on a
  non-symmetric mask with its transposed list, through the C ABI with the map from
  fwn_tiles_ds_map: equal bit for bit to the package's backward (which takes the same path),
  dK and dV equal to fwn_attn_bwd_launch's, all within the bars of the dense float64 oracle.
  The dS buffer starts as NaN bytes: every unit the dQ kernel reads was written."""
  rng = np.random.default_rng(66)
  b, n, h, d = 2, 700, 2, 128
  q, k, v, do = (rounded(rng.standard_normal((b, n, h, d)), dtype) for _ in range(4))
  m = random_mask(n, 0.05, 67, symmetric=False)
  cap, cap_t = (2, 3) if split else (1 << 20, 1 << 20)
  tiles = fwn.TileList.from_mask(m, max_item_tiles=cap)
  tiles_t = fwn.TileList.from_mask(m.T.tocsr(), max_item_tiles=cap_t)
  dmap = tiles.ds_map(tiles_t, fwn.hip_attn.unit_keys_for(dtype))
  assert dmap is not None and dmap.n_units > 0
  qd, kd, vd, dod = (dev(x, dtype) for x in (q, k, v, do))
  scale = d ** -0.5
  out, lse = fwn.attention_forward(qd, kd, vd, tiles, scale)
  desc = nat.AttnDesc(b, n, h, d, DT[dtype], scale, *qd.stride()[:3])
  size = _ws_size(desc, tiles, tiles_t)
  ws = torch.full((max(size, 1),), 255, dtype=torch.uint8, device="cuda")
  nbytes = dmap.ds_bytes(desc)
  assert nbytes == b * h * dmap.n_units * (1024 if dtype == torch.bfloat16 else 4096)
  ds = torch.full((nbytes,), 0xFF, dtype=torch.uint8, device="cuda")
  stream = torch.cuda.current_stream().cuda_stream
  L = nat.lib()

  def grads(ds_mode):
    delta = torch.full((b, h, n), float("nan"), device="cuda")
    dq, dk, dv = (torch.full_like(qd, float("nan")) for _ in range(3))
    if ds_mode:
      nat.check(L.fwn_attn_bwd_ds_launch(desc, qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), out.data_ptr(),
                                         dod.data_ptr(), lse.data_ptr(), delta.data_ptr(), tiles.struct,
                                         tiles_t.struct, dmap.struct, dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                                         ds.data_ptr(), nbytes, ws.data_ptr() if size else None, size, stream))
    else:
      nat.check(L.fwn_attn_bwd_launch(desc, qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), out.data_ptr(),
                                      dod.data_ptr(), lse.data_ptr(), delta.data_ptr(), tiles.struct, tiles_t.struct,
                                      dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), ws.data_ptr() if size else None,
                                      size, stream))
    return dq, dk, dv

  got = grads(True)
  recompute = grads(False)
  ref = fwn.attention_backward(qd, kd, vd, out, lse, dod, tiles, tiles_t, scale)
  torch.cuda.synchronize()
  for name, x, want in zip(("dq", "dk", "dv"), got, ref):
    np.testing.assert_array_equal(host(x), host(want), err_msg=name)
  for name, x, want in zip(("dk", "dv"), got[1:], recompute[1:]):
    np.testing.assert_array_equal(host(x), host(want), err_msg=name)
  dense = A.dense_grads(q, k, v, do, m.toarray(), scale)
  for name, x, want in zip(("dq", "dk", "dv"), got, dense):
    check(host(x), want, dtype, name)


@pytest.mark.parametrize("split", [False, True])
def test_bwd_ds_launch_bf16x3_one_stream(split):
  """The bf16x3 (split-precision) forward and dS-exchange backward through the C ABI on one
  stream, float32 tensors of a non-symmetric mask with its transposed list: equal bit for bit to
  the package's path (precision="bf16x3"), within rel RMS 1e-5 of the float64 oracle. The
  workspace starts as 0xFF bytes and the dS buffer as NaNs: every split row and unit read was
  written."""
  rng = np.random.default_rng(68)
  b, n, h, d = 2, 700, 2, 128
  q, k, v, do = (rng.standard_normal((b, n, h, d)).astype(np.float32) for _ in range(4))
  m = random_mask(n, 0.05, 69, symmetric=False)
  cap, cap_t = (2, 3) if split else (1 << 20, 1 << 20)
  tiles = fwn.TileList.from_mask(m, max_item_tiles=cap)
  tiles_t = fwn.TileList.from_mask(m.T.tocsr(), max_item_tiles=cap_t)
  dmap = tiles.ds_map(tiles_t, 32)
  qd, kd, vd, dod = (dev(x, torch.float32) for x in (q, k, v, do))
  scale = d ** -0.5
  desc = nat.AttnDesc(b, n, h, d, nat.F32, scale, *qd.stride()[:3], 0, 0, 0, nat.PREC_BF16X3, 0)
  size = _ws_size(desc, tiles, tiles_t)
  ws = torch.full((size,), 255, dtype=torch.uint8, device="cuda")
  nbytes = dmap.ds_bytes(desc)
  ds = torch.full((nbytes,), 0xFF, dtype=torch.uint8, device="cuda")
  stream = torch.cuda.current_stream().cuda_stream
  L = nat.lib()
  out, lse = torch.full_like(qd, float("nan")), torch.full((b, h, n), float("nan"), device="cuda")
  nat.check(L.fwn_attn_fwd_launch(desc, qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), tiles.struct, out.data_ptr(),
                                  lse.data_ptr(), ws.data_ptr(), size, stream))
  delta = torch.full((b, h, n), float("nan"), device="cuda")
  dq, dk, dv = (torch.full_like(qd, float("nan")) for _ in range(3))
  nat.check(L.fwn_attn_bwd_ds_launch(desc, qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), out.data_ptr(),
                                     dod.data_ptr(), lse.data_ptr(), delta.data_ptr(), tiles.struct, tiles_t.struct,
                                     dmap.struct, dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), ds.data_ptr(), nbytes,
                                     ws.data_ptr(), size, stream))
  pout, plse = fwn.attention_forward(qd, kd, vd, tiles, scale, precision="bf16x3")
  ref = fwn.attention_backward(qd, kd, vd, pout, plse, dod, tiles, tiles_t, scale, precision="bf16x3")
  torch.cuda.synchronize()
  np.testing.assert_array_equal(host(out), host(pout))
  for name, x, want in zip(("dq", "dk", "dv"), (dq, dk, dv), ref):
    np.testing.assert_array_equal(host(x), host(want), err_msg=name)
  dense = m.toarray()
  for name, x, want in zip(("out", "dq", "dk", "dv"), (out, dq, dk, dv),
                           (A.dense_attention(q, k, v, dense, scale),) + A.dense_grads(q, k, v, do, dense, scale)):
    assert A.rel_rms(host(x), want) <= 1e-5 and A.max_rel_err(host(x), want) <= 2e-5, name


@pytest.mark.parametrize("mode", ["recompute", "ds", "bf16x3"])
def test_graph_capture_replays_match_eager(mode):
  """The launchers allocate nothing and never synchronise, so a caller may capture them. The
  forward and the one-stream backward (split schedules, so the combine passes are captured too;
  "ds": the backward with the dS exchange and its dS buffer; "bf16x3": float32 tensors in the
  split precision, whose split passes are captured too) are captured into one graph, which is
  replayed four times with new inputs written in place between replays (eager copies and fills,
  with synchronisations in between); every replay equals the eager launches on the same inputs
  bit for bit."""
  ds = mode != "recompute"
  rng = np.random.default_rng(64)
  b, n, h, d = 1, 600, 2, 64
  dtype = torch.float32 if mode == "bf16x3" else torch.bfloat16
  m = random_mask(n, 0.04, 65, symmetric=True)
  tiles = fwn.TileList.from_mask(m, max_item_tiles=2)
  assert tiles.n_split > 0
  q, k, v, do = (torch.empty((b, n, h, d), dtype=dtype, device="cuda") for _ in range(4))
  scale = d ** -0.5
  if mode == "bf16x3":
    desc = nat.AttnDesc(b, n, h, d, nat.F32, scale, *q.stride()[:3], 0, 0, 0, nat.PREC_BF16X3, 0)
  else:
    desc = nat.AttnDesc(b, n, h, d, nat.BF16, scale, *q.stride()[:3])
  size = _ws_size(desc, tiles)
  dmap = tiles.ds_map(tiles, 32 if mode == "bf16x3" else 16)
  ds_bytes = dmap.ds_bytes(desc)
  L = nat.lib()

  def buffers():
    return dict(out=torch.empty_like(q), lse=torch.empty((b, h, n), device="cuda"),
                delta=torch.empty((b, h, n), device="cuda"), dq=torch.empty_like(q), dk=torch.empty_like(q),
                dv=torch.empty_like(q), ws=torch.empty(size, dtype=torch.uint8, device="cuda"),
                ds=torch.empty(ds_bytes, dtype=torch.uint8, device="cuda"))

  def launch(o, stream):
    nat.check(L.fwn_attn_fwd_launch(desc, q.data_ptr(), k.data_ptr(), v.data_ptr(), tiles.struct, o["out"].data_ptr(),
                                    o["lse"].data_ptr(), o["ws"].data_ptr(), size, stream))
    if ds:
      nat.check(L.fwn_attn_bwd_ds_launch(desc, q.data_ptr(), k.data_ptr(), v.data_ptr(), o["out"].data_ptr(),
                                         do.data_ptr(), o["lse"].data_ptr(), o["delta"].data_ptr(), tiles.struct,
                                         None, dmap.struct, o["dq"].data_ptr(), o["dk"].data_ptr(), o["dv"].data_ptr(),
                                         o["ds"].data_ptr(), ds_bytes, o["ws"].data_ptr(), size, stream))
      return
    nat.check(L.fwn_attn_bwd_launch(desc, q.data_ptr(), k.data_ptr(), v.data_ptr(), o["out"].data_ptr(),
                                    do.data_ptr(), o["lse"].data_ptr(), o["delta"].data_ptr(), tiles.struct, None,
                                    o["dq"].data_ptr(), o["dk"].data_ptr(), o["dv"].data_ptr(), o["ws"].data_ptr(),
                                    size, stream))

  def fill_inputs(seed):
    r = np.random.default_rng(seed)
    for t in (q, k, v, do):
      t.copy_(torch.from_numpy(r.standard_normal((b, n, h, d)).astype(np.float32)).to("cuda"))

  fill_inputs(0)
  captured, eager = buffers(), buffers()
  launch(eager, torch.cuda.current_stream().cuda_stream)  # loads the kernels before the capture
  torch.cuda.synchronize()
  graph = torch.cuda.CUDAGraph()
  with torch.cuda.graph(graph):
    launch(captured, torch.cuda.current_stream().cuda_stream)
  torch.cuda.synchronize()
  for replay in range(4):
    fill_inputs(100 + replay)
    for t in captured.values():
      if t.dtype != torch.uint8:
        t.fill_(float("nan"))
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    launch(eager, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    for name in ("out", "lse", "delta", "dq", "dk", "dv"):
      np.testing.assert_array_equal(host(captured[name]), host(eager[name]), err_msg=f"replay {replay} {name}")
    ref = A.dense_attention(*(host(t) for t in (q, k, v)), m.toarray(), scale)
    check(host(captured["out"]), ref, torch.bfloat16 if mode == "bf16x3" else dtype, ("replay", replay))
