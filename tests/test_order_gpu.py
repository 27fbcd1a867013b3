"""Order tables on the GPU: every kernel that decodes a job from its workgroup id (bf16, float32
and bf16x3 forwards, the dS-exchange and recomputing backwards, including the float32 and
bf16x3 dK/dV kernels that run two workgroups per item) gives, under each order of
fwn_tiles_order_fill, the same bits as without a table: the jobs, their partial slots and the
combine order are the same, only the workgroups that run them change. Padding entries exit
without writing. The library's own choice for bf16 calls is checked against the dense float64
oracle (oracle/attention.py)."""
import ctypes

import numpy as np
import pytest
import torch

import faster_weathernext_amd as fwn
from faster_weathernext_amd import _native as nat
from oracle import attention as A
from gpu_helpers import DEV, TOL, MAXTOL, random_mask, rounded, dev, host

pytestmark = pytest.mark.gpu

ORDERS = [(nat.ORDER_ITEMS, 0), (nat.ORDER_BALANCED, 0), (nat.ORDER_BALANCED, 128), (nat.ORDER_ITEMS, 5),
          (nat.ORDER_MAKESPAN, 64)]


def _workspace(desc, struct):
  size = ctypes.c_uint64(0)
  nat.check(nat.lib().fwn_attn_workspace_size(desc, struct, ctypes.byref(size)))
  return torch.empty(max(int(size.value), 256), dtype=torch.uint8, device=DEV)


def _run(struct, tiles, q, k, v, do, scale, precision, recompute):
  """Forward, the dS-exchange backward and (native precision) the recomputing backward under
  schedule `struct` of `tiles` (a symmetric mask): every output on the host."""
  L = nat.lib()
  stream = torch.cuda.current_stream().cuda_stream
  dt = nat.BF16 if q.dtype == torch.bfloat16 else nat.F32
  desc = nat.AttnDesc(q.shape[0], q.shape[1], q.shape[2], q.shape[3], dt, scale, *q.stride()[:3], 0, 0, 0,
                      precision, 0)
  native = nat.AttnDesc(q.shape[0], q.shape[1], q.shape[2], q.shape[3], dt, scale, *q.stride()[:3])
  ws = _workspace(desc, struct)
  out = torch.empty_like(q)
  lse = torch.empty((q.shape[0], q.shape[2], q.shape[1]), dtype=torch.float32, device=DEV)
  nat.check(L.fwn_attn_fwd_launch(desc, q.data_ptr(), k.data_ptr(), v.data_ptr(), struct, out.data_ptr(),
                                  lse.data_ptr(), ws.data_ptr(), ws.numel(), stream))
  dmap = tiles.ds_map(tiles, 16 if dt == nat.BF16 else 32)
  ds = torch.empty(max(dmap.ds_bytes(desc), 256), dtype=torch.uint8, device=DEV)
  delta = torch.empty_like(lse)
  res = {"out": out, "lse": lse}
  g = [torch.empty_like(q) for _ in range(3)]
  nat.check(L.fwn_attn_bwd_ds_launch(desc, q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), do.data_ptr(),
                                     lse.data_ptr(), delta.data_ptr(), struct, struct, dmap.struct, g[0].data_ptr(),
                                     g[1].data_ptr(), g[2].data_ptr(), ds.data_ptr(), ds.numel(), ws.data_ptr(),
                                     ws.numel(), stream))
  res.update(dq=g[0], dk=g[1], dv=g[2])
  if recompute:
    r = [torch.empty_like(q) for _ in range(3)]
    nat.check(L.fwn_attn_bwd_launch(native, q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), do.data_ptr(),
                                    lse.data_ptr(), delta.data_ptr(), struct, struct, r[0].data_ptr(),
                                    r[1].data_ptr(), r[2].data_ptr(), ws.data_ptr(), ws.numel(), stream))
    res.update(dq_recompute=r[0], dk_recompute=r[1], dv_recompute=r[2])
  torch.cuda.synchronize()
  return {name: host(t) for name, t in res.items()}


@pytest.mark.parametrize("case", ["bf16", "f32", "bf16x3"])
@pytest.mark.parametrize("cap", [0, 3])
def test_every_order_gives_the_plain_order_bits(cap, case):
  rng = np.random.default_rng(80 + cap)
  b, n, h, d = 2, 1100, 3, 64
  dtype = torch.bfloat16 if case == "bf16" else torch.float32
  precision = nat.PREC_BF16X3 if case == "bf16x3" else nat.PREC_NATIVE
  q, k, v, do = (rounded(rng.standard_normal((b, n, h, d)), dtype) for _ in range(4))
  m = random_mask(n, 0.03, 81, symmetric=True).tolil()
  for r in (3, 700):  # rows without keys
    m[r, :] = False
    m[:, r] = False
  m = m.tocsr()
  m.eliminate_zeros()
  tiles = fwn.TileList(*fwn.build_tile_mask(m), n, DEV, cap or None)
  sch = tiles.schedule_for(b, h)
  if cap:
    assert sch.n_split > 0
  args = [dev(x, dtype) for x in (q, k, v, do)]
  want = _run(sch.struct, tiles, *args, d ** -0.5, precision, precision == nat.PREC_NATIVE)
  for order, window in ORDERS:
    st = sch.ordered_struct(b * h, order, window, 32)
    table = sch.order_table(b * h, order, window, 32)
    assert st.n_work == len(table) >= sch.n_items * b * h
    print(f"{case} cap {cap} order {order} window {window}: {st.n_work} entries", flush=True)
    got = _run(st, tiles, *args, d ** -0.5, precision, precision == nat.PREC_NATIVE)
    for name in want:
      np.testing.assert_array_equal(got[name], want[name], err_msg=f"{name} order {order} window {window}")


@pytest.mark.parametrize("b,h,n", [(1, 1, 200), (1, 2, 642), (4, 4, 700), (3, 5, 1300)])
def test_orders_at_edge_shapes(b, h, n):
  """Order tables where most XCDs get one job or none (a 2-block list, one pair), odd pair
  counts and more pairs than XCDs: the bf16 forward and dS-exchange backward give the plain
  order's bits under every order."""
  rng = np.random.default_rng(100 + n)
  d = 64
  q, k, v, do = (rounded(rng.standard_normal((b, n, h, d)), torch.bfloat16) for _ in range(4))
  m = random_mask(n, 0.05, 101, symmetric=True)
  tiles = fwn.TileList(*fwn.build_tile_mask(m), n, DEV)
  sch = tiles.schedule_for(b, h)
  args = [dev(x, torch.bfloat16) for x in (q, k, v, do)]
  want = _run(sch.struct, tiles, *args, d ** -0.5, nat.PREC_NATIVE, True)
  for order, window in ORDERS:
    st = sch.ordered_struct(b * h, order, window, 32)
    print(f"b {b} h {h} n {n} order {order} window {window}: {st.n_work} entries for {sch.n_items * b * h} jobs",
          flush=True)
    got = _run(st, tiles, *args, d ** -0.5, nat.PREC_NATIVE, True)
    for name in want:
      np.testing.assert_array_equal(got[name], want[name], err_msg=f"{name} order {order} window {window}")


def test_library_orders_bf16_calls_and_matches_the_oracle():
  """The op's bf16 calls with few jobs launch with the order tables (windows of
  hip_attn.ORDER_WINDOWS); the result is the plain order's bit for bit and within the bf16 bars
  of the dense oracle."""
  rng = np.random.default_rng(90)
  b, n, h, d = 1, 2000, 2, 64
  q, k, v, do = (rounded(rng.standard_normal((b, n, h, d)), torch.bfloat16) for _ in range(4))
  m = random_mask(n, 0.02, 91, symmetric=True)
  tiles = fwn.TileList(*fwn.build_tile_mask(m), n, DEV)
  st = tiles.struct_for(b, h, (nat.ORDER_BALANCED, fwn.hip_attn.ORDER_WINDOWS["bf16"]["fwd"], 64))
  assert tiles.order_for(b, h) and st.n_work > 0 and st.work_pairs == b * h
  args = [dev(x, torch.bfloat16, grad=True) for x in (q, k, v)]
  out = fwn.tiled_flash_attention(*args, tiles, scale=d ** -0.5)
  out.backward(dev(do, torch.bfloat16))
  plain = _run(tiles.schedule_for(b, h).struct, tiles, *(a.detach() for a in args), dev(do, torch.bfloat16),
               d ** -0.5, nat.PREC_NATIVE, False)
  np.testing.assert_array_equal(host(out), plain["out"])
  for t, name in zip(args, ("dq", "dk", "dv")):
    np.testing.assert_array_equal(host(t.grad), plain[name])
  mask = m.toarray()
  want = A.dense_attention(q, k, v, mask, d ** -0.5)
  grads = A.dense_grads(q, k, v, do, mask, d ** -0.5)
  for got, ref, name in [(host(out), want, "out")] + [(host(t.grad), r, nm) for t, r, nm in
                                                        zip(args, grads, ("dq", "dk", "dv"))]:
    rel = np.sqrt(np.mean((got - ref) ** 2)) / np.sqrt(np.mean(ref ** 2))
    mx = np.abs(got - ref).max() / np.abs(ref).max()
    assert rel < TOL[torch.bfloat16] and mx < MAXTOL[torch.bfloat16], (name, rel, mx)
