"""Block-sparse masked flash attention on MI355X: the public op and its tile lists.

Mirrors the reference's ``faster_weathernext.pallas_attn`` (``pallas_attn.py:317-354``):

    out = tiled_flash_attention(q, k, v, tile_ptr, tile_kb, tile_bits, scale=D**-0.5, tiles_t=None)

with q, k, v [batch, n, heads, head_dim] (torch tensors on the GPU, float32 or bfloat16), the tile
list from ``build_tile_mask`` (128 x 128 tiles here, 64 x 32 in the reference) and the same
gradient contract: differentiable with respect to q, k, v; the dK/dV kernel walks ``tiles_t``, the
transposed mask's tile list, which defaults to the forward list (right for symmetric masks such as
k-hop neighbourhoods). The reference's Pallas knobs (block_q, block_k, num_warps, num_stages,
bwd_num_warps, bwd_split, interpret) have no counterpart: tile shape and wave count are fixed by
the gfx950 kernels, and there is no interpreter or CPU path.

All compute runs in the HIP kernels of libfwn_attn.so through its C ABI; torch only provides
device memory and the stream. Tensors must be on a ROCm device: there is no CPU fallback.
"""
import collections
import ctypes
import threading
import weakref

import numpy as np
import torch

from . import _native as nat
from .mesh import build_tile_mask, hilbert_order  # noqa: F401  (re-exported, as in the reference module)

BLOCK_Q = nat.BLOCK
BLOCK_K = nat.BLOCK

_DTYPES = {torch.float32: nat.F32, torch.bfloat16: nat.BF16}


# Work items (split-K): each block's run of live tiles is cut into items of at most a cap. A long
# cap leaves fewer partial results to combine; a short one balances the launch better when there
# are few jobs. With no cap given, a TileList picks per launch from the unsplit job count
# blocks x batch x heads: WIDE_ITEM_TILES from WIDE_JOBS (6 jobs per CU of the 256) up, else
# nat.ITEM_TILES. Measured on MI355X (TFLOP/s): C3 (1,284 jobs) 1063 at 64 against 1028 at 96;
# C5 forward (1,926 jobs) 0.903 ms at 64 against 0.870 at 128; C4 (10,272 jobs) 1435 at 64
# against 1458 at 128.
WIDE_ITEM_TILES = 128
WIDE_JOBS = 1536

# Order tables (fwn_tiles_order_fill) for calls whose per-item launch has fewer than ORDER_JOBS
# jobs: each XCD takes a contiguous range of equal estimated cost, run longest first within
# windows of ORDER_WINDOWS[products][kernel] jobs counted from the range's end (0: the range in
# block order). A window is one round of an XCD's slots: 64 jobs for the forward and dQ (two
# workgroups per CU, 32 CUs per XCD), 32 for dK/dV (one per CU). Measured on MI355X (two or
# three runs each on one box):
#   bf16 fwd+bwd, plain order -> tables: C3 1.562 -> 1.496 ms and the C5 attention shape
#     2.897 -> 2.852 ms with windows of two rounds counted from the start; counted from the end,
#     C3 1.48 -> 1.44 ms, C5 unchanged; then one round (64 / 64 / 32 against 128 / 128 / 64):
#     C3 1.323 -> 1.292 ms, C5 2.775 -> 2.72 ms. Windows of 48 / 48 / 24 and 32 / 32 / 16 were
#     slower (C3 1.367, 1.356 ms).
#   float32 (IEEE products): C2 forward 2.21 -> 1.92 ms; C5 shape fwd+bwd 19.40 -> 18.32 ms.
#   bf16x3 products: C2 forward 0.764 -> 0.62 ms; at the C5 shape windows made dQ 5% slower, so
#     dQ takes equal-cost ranges alone (step 7.00 -> 6.86 ms).
# Sorting whole ranges, or all jobs, longest first lost the neighbouring blocks' shared K/V and
# dS reads (C5 dQ +4-30%). With many jobs per slot (C4's 10,464) the plain ranges are already
# even, so such calls keep the plain order.
ORDER_JOBS = 4096
ORDER_WINDOWS = {"bf16": {"fwd": 64, "dq": 64, "kv": 32},
                 "f32": {"fwd": 64, "dq": 64, "kv": 32},
                 "bf16x3": {"fwd": 64, "dq": 0, "kv": 32}}
# How each kernel's ranges are cut (nat.ORDER_BALANCED: equal estimated cost; nat.ORDER_MAKESPAN:
# equal simulated end on ORDER_SLOTS[kernel] slots per XCD) and its workgroups per XCD. For
# dK/dV at C3 the equal-cost ranges left four XCDs with a last round of 7 jobs (199 on 32 slots)
# and four with a full one (191), ending 29 us apart; the simulated ends matched the measured
# ones (correlation 1.0), and cutting by them took dK/dV 0.668-0.670 -> 0.661-0.662 ms (C5 shape
# unchanged). For the forward and dQ the cost model misjudges C3's coarse-node items, and the
# simulated cut measured 1-2% slower.
ORDER_CUTS = {"fwd": nat.ORDER_BALANCED, "dq": nat.ORDER_BALANCED, "kv": nat.ORDER_MAKESPAN}
ORDER_SLOTS = {"fwd": 64, "dq": 64, "kv": 32}
# A job's estimated cost: ORDER_ITEM_UNITS, plus per tile ORDER_TILE_UNITS and ORDER_HALF_UNITS
# per live 32 x 16 half (the tile's set half bits). Fitted to per-workgroup durations at C3 and
# the C5 shape (the tile count alone misjudged C3's sparse coarse-node blocks; with the halves
# the predicted per-XCD work follows the measured XCD end times, correlation 0.9-1.0). Measured
# against tiles + 3 per item: C3 1.493 -> 1.482 ms, C5 shape 2.871 -> 2.868 ms.
ORDER_ITEM_UNITS = 20
ORDER_TILE_UNITS = 20
ORDER_HALF_UNITS = 1


def order_plan(desc, kernel):
  """(cut, window, slots) of the order table for `kernel` ("fwd", "dq" or "kv") of a call with
  descriptor `desc`."""
  if desc.precision == nat.PREC_BF16X3:
    products = "bf16x3"
  else:
    products = "bf16" if desc.dtype == nat.BF16 else "f32"
  return ORDER_CUTS[kernel], ORDER_WINDOWS[products][kernel], ORDER_SLOTS[kernel]


class _Schedule:
  """One split-K schedule of a TileList: its work items, split records and C struct, plus the
  order tables built for it (``ordered_struct``)."""

  def __init__(self, tl, tile_ptr, cap):
    L = nat.lib()
    counts = np.zeros(3, np.int32)
    nat.check(L.fwn_tiles_schedule_count(tl.n_blocks, nat.ptr(tile_ptr), int(cap), nat.ptr(counts[0:]),
                                         nat.ptr(counts[1:]), nat.ptr(counts[2:])))
    self.n_items, self.n_parts, self.n_split = (int(c) for c in counts)
    items = np.zeros((self.n_items, 4), np.int32)
    split = np.zeros((max(self.n_split, 1), 3), np.int32)
    nat.check(L.fwn_tiles_schedule_fill(tl.n_blocks, nat.ptr(tile_ptr), int(cap), nat.ptr(items), nat.ptr(split)))
    self.items_host = items
    self.split_host = split[:self.n_split]
    self.items = torch.from_numpy(items).to(tl.device)
    self.split = torch.from_numpy(split).to(tl.device)
    self._tl = tl
    self._orders = {}
    self.struct = self._struct()

  def _struct(self, work=None, pairs=0):
    addr = lambda t: t.data_ptr() if t is not None and t.numel() else None
    tl = self._tl
    return nat.Tiles(tl.n_blocks, tl.n_tiles, addr(tl.ptr), addr(tl.col), addr(tl.lanes), addr(tl.groups),
                     self.n_items, self.n_parts, self.n_split, 0 if work is None else work.shape[0],
                     addr(self.items), addr(self.split) if self.n_split else None, addr(tl.halves), addr(work),
                     pairs, 0)

  def order_table(self, pairs, order=nat.ORDER_BALANCED, window=0, slots=64):
    """Host order table [n_work, 2] of this schedule for calls of `pairs` (batch, head) pairs."""
    L = nat.lib()
    n = np.zeros(1, np.int32)
    halves = np.unpackbits(self._tl.halves_host.astype("<u4").view(np.uint8).reshape(-1, 4), axis=1).sum(1)
    cost = (ORDER_TILE_UNITS + ORDER_HALF_UNITS * halves).astype(np.int32)
    args = (self.n_items, nat.ptr(self.items_host), nat.ptr(cost) if len(cost) else None, ORDER_ITEM_UNITS,
            int(pairs), int(order), int(window), int(slots))
    nat.check(L.fwn_tiles_order_count(*args, nat.ptr(n)))
    work = np.zeros((int(n[0]), 2), np.int32)
    nat.check(L.fwn_tiles_order_fill(*args, nat.ptr(work)))
    return work

  def ordered_struct(self, pairs, order=nat.ORDER_BALANCED, window=0, slots=64):
    """The C struct with an order table for calls of `pairs` (batch, head) pairs (built once)."""
    key = (int(pairs), int(order), int(window), int(slots))
    if key not in self._orders:
      work = torch.from_numpy(self.order_table(pairs, order, window, slots)).to(self._tl.device)
      self._orders[key] = (work, self._struct(work, int(pairs)))
    return self._orders[key][1]


class TileList:
  """A tile list prepared for the kernels and resident on one device.

  Built from the canonical arrays of ``build_tile_mask`` (validated on the host, converted to the
  kernels' per-lane mask layout by ``fwn_tiles_prepare`` and copied once), then shared by every
  call, as the reference shares one device copy of the mask across layers (``patch.py:263-266``).
  ``max_item_tiles`` fixes the split-K cap; None lets each launch pick it (``struct_for``).
  ``struct`` is the schedule with the fixed cap, or nat.ITEM_TILES.
  """

  def __init__(self, tile_ptr, tile_kb, tile_bits, n_cols, device="cuda", max_item_tiles=None):
    tile_ptr = nat.as_c(tile_ptr, np.int32)
    tile_kb = nat.as_c(tile_kb, np.int32)
    tile_bits = nat.as_c(tile_bits, np.uint32)
    if tile_ptr.ndim != 1 or tile_kb.ndim != 1 or len(tile_ptr) < 1:
      raise ValueError("tile_ptr and tile_kb must be 1-D int32 arrays (tile_ptr of length n_blocks + 1)")
    want = (len(tile_kb), nat.BLOCK, nat.BLOCK // 32)
    if tile_bits.size != int(np.prod(want)):
      # The reference's own lists are 64 x 32 tiles (uint32[T, 64], pallas_attn.py:93); these
      # kernels take 128 x 128 tiles only (uint32[T, 128, 4]), from this package's build_tile_mask.
      raise ValueError(f"tile_bits has shape {tuple(tile_bits.shape)}; expected {want}: 128 x 128 tiles "
                       "(bit j of word w of row r = key 32w + j), as build_tile_mask here writes them")
    tile_bits = tile_bits.reshape(want)
    self.n_blocks = len(tile_ptr) - 1
    self.n_tiles = len(tile_kb)
    self.n_cols = int(n_cols)
    L = nat.lib()
    lanes = np.zeros((self.n_tiles, nat.LANE_WORDS), np.uint64)
    groups = np.zeros(self.n_tiles, np.uint32)
    halves = np.zeros(self.n_tiles, np.uint32)
    nat.check(L.fwn_tiles_prepare(self.n_blocks, self.n_tiles, self.n_cols, nat.ptr(tile_ptr), nat.ptr(tile_kb),
                                  nat.ptr(tile_bits), nat.ptr(lanes), nat.ptr(groups), nat.ptr(halves)))
    self.device = torch.device(device)
    put = lambda a: torch.from_numpy(a).to(self.device)
    self.ptr = put(tile_ptr)
    self.col = put(tile_kb)
    self.lanes = put(lanes.view(np.int64))
    self.groups = put(groups.view(np.int32))
    self.groups_host = groups
    self.halves = put(halves.view(np.int32))
    self.halves_host = halves
    self.counts = np.diff(tile_ptr)
    self.nnz = int(np.unpackbits(tile_bits.view(np.uint8)).sum()) if self.n_tiles else 0
    self._tile_ptr = tile_ptr
    self._tile_col = tile_kb
    self._tile_bits = tile_bits
    self._ds_maps = {}
    self._fixed_cap = None if max_item_tiles is None else int(max_item_tiles)
    self._schedules = {}
    base = self._schedule(nat.ITEM_TILES if self._fixed_cap is None else self._fixed_cap)
    self.n_items, self.n_parts, self.n_split = base.n_items, base.n_parts, base.n_split
    self.items_host, self.split_host = base.items_host, base.split_host
    self.items, self.split = base.items, base.split
    self.struct = base.struct

  def _schedule(self, cap):
    cap = int(cap) if cap > 0 else nat.ITEM_TILES
    if cap not in self._schedules:
      self._schedules[cap] = _Schedule(self, self._tile_ptr, cap)
    return self._schedules[cap]

  def item_cap_for(self, batch, heads, kernel="fwd"):
    """Longest run of tiles per work item for `kernel` ("fwd", "dq" or "kv") of a call of
    `batch` x `heads`: the cap fixed at construction, else WIDE_ITEM_TILES for dK/dV and for the
    others from WIDE_JOBS jobs up, nat.ITEM_TILES below. With the order tables, C3 (1,284 jobs)
    measured dK/dV 0.663 ms at 64, 0.660 at 96 or 128 and 0.693 at 160 (step 1.331 -> 1.326
    ms), and the forward 0.398 ms at 64 against 0.415 at 128."""
    if self._fixed_cap is not None:
      return self._fixed_cap if self._fixed_cap > 0 else nat.ITEM_TILES
    wide = kernel == "kv" or self.n_blocks * int(batch) * int(heads) >= WIDE_JOBS
    return WIDE_ITEM_TILES if wide else nat.ITEM_TILES

  def schedule_for(self, batch, heads, kernel="fwd"):
    """The split-K schedule `kernel` of a call of `batch` x `heads` launches (items, split blocks,
    C struct)."""
    return self._schedule(self.item_cap_for(batch, heads, kernel))

  def order_for(self, batch, heads, kernel="fwd"):
    """Whether `kernel` of a call of `batch` x `heads` takes an order table: fewer than
    ORDER_JOBS jobs in its per-item launch."""
    sch = self.schedule_for(batch, heads, kernel)
    return sch.n_items * int(batch) * int(heads) < ORDER_JOBS

  def struct_for(self, batch, heads, plan=None, kernel="fwd"):
    """The C struct to launch `kernel` of a call of `batch` x `heads` with (the schedule chosen
    for it); with a `plan` (cut, window, slots) and few jobs (``order_for``), with that order
    table."""
    sch = self.schedule_for(batch, heads, kernel)
    if plan is not None and self.order_for(batch, heads, kernel):
      return sch.ordered_struct(int(batch) * int(heads), *plan)
    return sch.struct

  def struct_for_desc(self, desc, kernel="fwd"):
    """The C struct for `kernel` ("fwd", "dq", or "kv" for dK/dV with this list as the transposed
    list) of a call with descriptor `desc`."""
    return self.struct_for(desc.batch, desc.heads, order_plan(desc, kernel), kernel)

  def workspace_bytes(self, desc):
    """Workspace the launchers need for this list and the call shape `desc`: the most any of
    the schedules ``struct_for_desc`` picks for its kernels needs (0 if none splits a block)."""
    n = ctypes.c_uint64(0)
    most = 0
    for kernel in ("fwd", "dq", "kv"):
      nat.check(nat.lib().fwn_attn_workspace_size(desc, self.struct_for_desc(desc, kernel), ctypes.byref(n)))
      most = max(most, int(n.value))
    return most

  def ds_map(self, tiles_t, unit_keys=16):
    """The dS exchange's unit numbering of this (forward) list and `tiles_t` (this list itself
    for a symmetric mask) for units of `unit_keys` keys (16 for bf16, 32 for float32), or None
    when `tiles_t` is not this list's exact transpose; built on first use and kept with this
    list."""
    # Weakly keyed by the transposed list: a map lives only as long as its tiles_t (which may be
    # this list), so lists evicted from _as_tiles' cache take their maps with them.
    maps = self._ds_maps.setdefault(int(unit_keys), weakref.WeakKeyDictionary())
    if tiles_t not in maps:
      maps[tiles_t] = DsMap.build(self, tiles_t, unit_keys)
    return maps[tiles_t]

  @classmethod
  def from_mask(cls, mask, perm=None, device="cuda", max_item_tiles=None):
    """Tile list of a boolean scipy/numpy [n, n] mask (optionally permuted as mask[perm][:, perm])."""
    tp, kb, bits = build_tile_mask(mask, perm=perm)
    return cls(tp, kb, bits, mask.shape[1], device, max_item_tiles)

  @property
  def density(self):
    """Fraction of valid entries in the live tiles."""
    return self.nnz / max(1, self.n_tiles * nat.BLOCK * nat.BLOCK)

  @property
  def group_fraction(self):
    """Fraction of the live tiles' 32 x 32 groups that hold a valid element: the share of the
    live-tile work the kernels execute (the other groups are skipped)."""
    if not self.n_tiles:
      return 0.0
    bits = np.unpackbits((self.groups_host & 0xFFFF).astype('<u4').view(np.uint8)).sum()
    return float(bits) / (16 * self.n_tiles)


class DsMap:
  """Unit numbering of the backward's dS exchange (``fwn_tiles_ds_map``): the dK/dV kernel writes
  each unit of dS = P (dP - delta) once, and the dQ kernel reads it instead of recomputing S and
  dP (5 contractions per live tile instead of 7). A unit is 32 queries x `unit_keys` keys: 16
  (bf16, the set bits of the forward list's half words) or 32 (float32, its group bits),
  numbered tile by tile; ``struct`` is the C view."""

  def __init__(self, n_units, ubase, tmap, unit_keys, device):
    self.n_units = int(n_units)
    self.unit_keys = int(unit_keys)
    self.ubase = torch.from_numpy(ubase).to(device)
    self.tmap = torch.from_numpy(tmap).to(device)
    addr = lambda t: t.data_ptr() if t.numel() else None
    self.struct = nat.DsMap(self.n_units, addr(self.ubase), addr(self.tmap), self.unit_keys, 0)

  @classmethod
  def build(cls, tl, tlt, unit_keys=16):
    """The map of forward list `tl` and transposed list `tlt`, or None if `tlt` is not the
    transpose of `tl` bit for bit (the recomputing backward applies then)."""
    if tl.n_blocks != tlt.n_blocks or tl.n_cols != tlt.n_cols or tl.device != tlt.device:
      return None
    ubase = np.zeros(max(tl.n_tiles, 1), np.int32)
    tmap = np.zeros((max(tlt.n_tiles, 1), 2), np.int32)
    n_units = np.zeros(1, np.int64)
    status = nat.lib().fwn_tiles_ds_map(tl.n_blocks, nat.ptr(tl._tile_ptr), nat.ptr(tl._tile_col),
                                        nat.ptr(tl._tile_bits), nat.ptr(tlt._tile_ptr), nat.ptr(tlt._tile_col),
                                        nat.ptr(tlt._tile_bits), int(unit_keys), nat.ptr(ubase), nat.ptr(tmap),
                                        nat.ptr(n_units))
    if status == nat.ERR_TILES:
      return None
    nat.check(status)
    return cls(n_units[0], ubase[:tl.n_tiles], tmap[:tlt.n_tiles], unit_keys, tl.device)

  def ds_bytes(self, desc):
    n = ctypes.c_uint64(0)
    nat.check(nat.lib().fwn_attn_ds_bytes(desc, self.struct, ctypes.byref(n)))
    return int(n.value)


# The backward uses the dS exchange (DsMap) when the lists allow it; False keeps the
# recomputing dQ kernel beside dK/dV for every call.
DS_EXCHANGE = True


def unit_keys_for(dtype):
  """Keys per dS unit of the exchange for a dtype: 16 for bf16, 32 for float32."""
  return 16 if dtype == torch.bfloat16 else 32

_cache_lock = threading.Lock()
_cache = collections.OrderedDict()
# Prepared lists kept for array triples passed directly to the op (least recently used first out).
# Each holds its device arrays (about 38 MB at refinement 6, 32-hop); callers that build arrays
# anew for every call should build a TileList once and pass that instead.
CACHE_LISTS = 4


def _as_tiles(tiles, n, device):
  """A TileList from a TileList or a (tile_ptr, tile_kb, tile_bits) tuple (prepared once, cached).

  A TileList is checked against the call: its column count must be n (a list built for more
  columns would address keys past n) and it must live on the call's device."""
  if isinstance(tiles, TileList):
    if tiles.n_cols != n:
      raise ValueError(f"tile list built for {tiles.n_cols} columns, but the call has n = {n} keys")
    if tiles.device.type != device.type or (tiles.device.index or 0) != (device.index or 0):
      raise ValueError(f"tile list lives on {tiles.device}, the tensors on {device}")
    return tiles
  tp, kb, bits = tiles
  key = (id(tp), id(kb), id(bits), n, str(device))
  with _cache_lock:
    hit = _cache.get(key)
    if hit is None or hit[0] is not tp or hit[1] is not kb or hit[2] is not bits:
      hit = (tp, kb, bits, TileList(np.asarray(tp), np.asarray(kb), np.asarray(bits), n, device))
      _cache[key] = hit
    _cache.move_to_end(key)
    while len(_cache) > CACHE_LISTS:
      _cache.popitem(last=False)
    return hit[3]


def _check(q):
  if q.dtype not in _DTYPES:
    raise TypeError(f"unsupported dtype {q.dtype}: float32 or bfloat16")
  if q.device.type != "cuda":
    raise ValueError("tiled_flash_attention runs on the GPU only (tensors are on %s)" % q.device)
  if q.dim() != 4:
    raise ValueError("expected [batch, n, heads, head_dim]")


# Product precision of the kernels (the reference picks its dot algorithm from jax's default
# matmul precision and strict_fp32, pallas_attn.py:336-341):
#   "native": products in the tensors' dtype (IEEE float32 products for float32, the reference's
#             strict_fp32; bf16 products for bf16);
#   "bf16x3": float32 tensors, each product from bf16 parts, hi*hi + hi*lo + lo*hi (about 16
#             significant bits per operand; the role of the reference's 3xTF32 "highest" dots).
#             The backward runs in bf16x3 as well with the dS exchange; with lists that are not
#             exact transposes (or DS_EXCHANGE False) it is the recomputing IEEE float32 one.
PRECISIONS = {"native": nat.PREC_NATIVE, "bf16x3": nat.PREC_BF16X3}


def _precision(precision, dtype):
  if precision not in PRECISIONS:
    raise ValueError(f"precision {precision!r}: one of {sorted(PRECISIONS)}")
  if precision == "bf16x3" and dtype != torch.float32:
    raise TypeError("precision 'bf16x3' needs float32 tensors")
  return PRECISIONS[precision]


def _desc(q, scale, o=None, precision=nat.PREC_NATIVE):
  """Call descriptor: q's strides for q, k, v, dq, dk, dv and o's for o, dout (0 = the same)."""
  b, n, h, d = q.shape
  sb, sn, sh, _ = q.stride()
  osb = osn = osh = 0
  if o is not None and o.stride() != q.stride():
    osb, osn, osh, _ = o.stride()
  return nat.AttnDesc(b, n, h, d, _DTYPES[q.dtype], float(scale), sb, sn, sh, osb, osn, osh, precision, 0)


def _in_place(x):
  """x itself when the kernels can read it where it lies (head_dim contiguous, strides and base
  16-byte aligned), else a contiguous copy."""
  ok = (x.stride(-1) == 1 and x.data_ptr() % 16 == 0 and
        all(st >= 0 and (st * x.element_size()) % 16 == 0 for st in x.stride()[:3]))
  return x if ok else x.contiguous()


def _same_layout(x, ref, name):
  """x in ref's strides (the kernels share one set of strides over q, k, v)."""
  if x.shape != ref.shape or x.dtype != ref.dtype or x.device != ref.device:
    raise ValueError(f"{name} must match q in shape, dtype and device")
  if x.stride() == ref.stride():
    return x
  y = torch.empty_strided(ref.shape, ref.stride(), dtype=ref.dtype, device=ref.device)
  y.copy_(x)
  return y


def _stream(device):
  return torch.cuda.current_stream(device).cuda_stream


def workspace(desc, device, *lists):
  """A device workspace large enough for every tile list in `lists` (None if none needs one)."""
  size = max(tl.workspace_bytes(desc) for tl in lists)
  return torch.empty(size, dtype=torch.uint8, device=device) if size else None


def _ws_args(ws):
  return (ws.data_ptr(), ws.numel()) if ws is not None else (None, 0)


def attention_forward(q, k, v, tiles, scale, with_lse=True, precision="native"):
  """Forward kernel: returns (out, lse) with lse float32 [batch, heads, n] (None if not requested).

  q, k, v are read where they lie when their strides allow it (e.g. views of one fused
  projection); out is a new contiguous [batch, n, heads, head_dim] tensor. ``precision``: see
  PRECISIONS.
  """
  _check(q)
  prec = _precision(precision, q.dtype)
  q = _in_place(q)
  k = _same_layout(k, q, "k")
  v = _same_layout(v, q, "v")
  out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
  desc = _desc(q, scale, out, prec)
  tl = _as_tiles(tiles, q.shape[1], q.device)
  lse = torch.empty((q.shape[0], q.shape[2], q.shape[1]), dtype=torch.float32, device=q.device) if with_lse else None
  ws = workspace(desc, q.device, tl)
  ts = tl.struct_for_desc(desc, "fwd")
  nat.check(nat.lib().fwn_attn_fwd_launch(desc, q.data_ptr(), k.data_ptr(), v.data_ptr(), ts, out.data_ptr(),
                                          lse.data_ptr() if with_lse else None, *_ws_args(ws), _stream(q.device)))
  return out, lse


_side_lock = threading.Lock()
_side_streams = {}


def _side_stream(device):
  """One extra stream per device (default priority) for the dK/dV kernel."""
  with _side_lock:
    s = _side_streams.get(device.index)
    if s is None:
      s = _side_streams[device.index] = torch.cuda.Stream(device)
  return s


def _backward_into(q, k, v, out, lse, dout, tiles, tiles_t, scale, dq, dk, dv, precision="native"):
  """Backward kernels writing dq, dk, dv (q's strides).

  With `tiles_t` the exact transpose of `tiles` (a symmetric mask with tiles_t None included):
  the dS exchange, in stream order on the current stream (fwn_attn_bwd_ds_launch): delta, dK/dV
  writing every unit of dS (32 x 16 in bf16, 32 x 32 in float32), then dQ from dS. The
  reference computes S and dP in both of its backward kernels (pallas_attn.py:172-180,
  199-207); here once (bf16 C3: 1.71 -> 1.58 ms per fwd+bwd step, C4 7.87 -> 6.97 ms).

  Otherwise (lists that are not transposes, DS_EXCHANGE False): the delta pre-pass, then the
  recomputing dQ kernel on the current stream and dK/dV on a side stream at the same time (each
  with its own workspace), joined before returning. Run side by side, each fills the CUs the
  other's last workgroups leave idle. The sequence is what fwn_attn_bwd_launch enqueues on one
  stream, with the dQ and dK/dV launches overlapped. ``precision`` "bf16x3" applies to the dS
  exchange only."""
  desc = _desc(q, scale, out)
  n = q.shape[1]
  tl = _as_tiles(tiles, n, q.device)
  tlt = tl if tiles_t is None else _as_tiles(tiles_t, n, q.device)
  delta = torch.empty_like(lse)
  L = nat.lib()
  main = torch.cuda.current_stream(q.device)
  dmap = tl.ds_map(tlt, unit_keys_for(q.dtype)) if DS_EXCHANGE else None
  if dmap is not None:
    # delta, dK/dV writing dS, then dQ from dS, in stream order (fwn_attn_bwd_ds_launch).
    desc = _desc(q, scale, out, _precision(precision, q.dtype))
    ws = workspace(desc, q.device, tl, tlt)
    ds = torch.empty(max(dmap.ds_bytes(desc), 256), dtype=torch.uint8, device=q.device)
    ts, tst = tl.struct_for_desc(desc, "dq"), tlt.struct_for_desc(desc, "kv")
    nat.check(L.fwn_attn_bwd_ds_launch(desc, q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                                       dout.data_ptr(), lse.data_ptr(), delta.data_ptr(), ts, tst, dmap.struct,
                                       dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), ds.data_ptr(), ds.numel(),
                                       *_ws_args(ws), main.cuda_stream))
    return
  ws_q, ws_kv = workspace(desc, q.device, tl), workspace(desc, q.device, tlt)
  nat.check(L.fwn_attn_bwd_delta_launch(desc, out.data_ptr(), dout.data_ptr(), delta.data_ptr(), main.cuda_stream))
  side = _side_stream(q.device)
  side.wait_stream(main)
  ts, tst = tl.struct_for_desc(desc, "dq"), tlt.struct_for_desc(desc, "kv")
  nat.check(L.fwn_attn_bwd_dkv_launch(desc, q.data_ptr(), k.data_ptr(), v.data_ptr(), dout.data_ptr(),
                                      lse.data_ptr(), delta.data_ptr(), tst, dk.data_ptr(), dv.data_ptr(),
                                      *_ws_args(ws_kv), side.cuda_stream))
  nat.check(L.fwn_attn_bwd_dq_launch(desc, q.data_ptr(), k.data_ptr(), v.data_ptr(), dout.data_ptr(),
                                     lse.data_ptr(), delta.data_ptr(), ts, dq.data_ptr(), *_ws_args(ws_q),
                                     main.cuda_stream))
  # Everything the side stream used was allocated on `main`; ordering main after it keeps the
  # caching allocator from handing those blocks out while the dK/dV kernel still runs.
  main.wait_stream(side)


def attention_backward(q, k, v, out, lse, dout, tiles, tiles_t, scale, precision="native"):
  """Backward kernels (delta pre-pass, dQ, dK/dV): returns contiguous (dq, dk, dv)."""
  _check(q)
  q = q.contiguous()  # dq, dk, dv are written in q's strides: keep them dense
  k = _same_layout(k, q, "k")
  v = _same_layout(v, q, "v")
  out = _in_place(out)
  dout = _same_layout(dout, out, "dout")
  dq, dk, dv = torch.empty_like(q), torch.empty_like(q), torch.empty_like(q)
  _backward_into(q, k, v, out, lse, dout, tiles, tiles_t, scale, dq, dk, dv, precision)
  return dq, dk, dv


class _TiledAttention(torch.autograd.Function):
  """custom VJP of the attention (``pallas_attn.py:260-311``): the forward saves q, k, v, out and
  the per-row log-sum-exp; the backward recomputes P tile by tile."""

  @staticmethod
  def forward(ctx, q, k, v, tiles, tiles_t, scale, precision):
    need = any(ctx.needs_input_grad[:3])
    out, lse = attention_forward(q, k, v, tiles, scale, with_lse=need, precision=precision)
    if need:
      ctx.save_for_backward(q, k, v, out, lse)
      ctx.tiles, ctx.tiles_t, ctx.scale, ctx.precision = tiles, tiles_t, scale, precision
    return out

  @staticmethod
  def backward(ctx, dout):
    q, k, v, out, lse = ctx.saved_tensors
    dq, dk, dv = attention_backward(q, k, v, out, lse, dout, ctx.tiles, ctx.tiles_t, ctx.scale, ctx.precision)
    return dq, dk, dv, None, None, None, None


class _TiledAttentionQKV(torch.autograd.Function):
  """The same custom VJP over one packed [batch, n, 3, heads, head_dim] q/k/v buffer: the kernels
  read q, k, v where the projection wrote them and write dq, dk, dv into one packed gradient."""

  @staticmethod
  def forward(ctx, qkv, tiles, tiles_t, scale, precision):
    q, k, v = qkv.unbind(2)
    need = ctx.needs_input_grad[0]
    out, lse = attention_forward(q, k, v, tiles, scale, with_lse=need, precision=precision)
    if need:
      ctx.save_for_backward(qkv, out, lse)
      ctx.tiles, ctx.tiles_t, ctx.scale, ctx.precision = tiles, tiles_t, scale, precision
    return out

  @staticmethod
  def backward(ctx, dout):
    qkv, out, lse = ctx.saved_tensors
    q, k, v = qkv.unbind(2)
    dqkv = torch.empty_like(qkv)
    dq, dk, dv = dqkv.unbind(2)
    _backward_into(q, k, v, out, lse, _same_layout(dout, out, "dout"), ctx.tiles, ctx.tiles_t, ctx.scale,
                   dq, dk, dv, ctx.precision)
    return dqkv, None, None, None, None


def tiled_flash_attention_qkv(qkv, tiles, *, scale, tiles_t=None, precision="native"):
  """Attention over a packed qkv [batch, n, 3, heads, head_dim] (one fused projection's output,
  contiguous) -> [batch, n, heads, head_dim], with no copy of q, k, v or of their gradients."""
  _check(qkv[:, :, 0])
  _precision(precision, qkv.dtype)
  if qkv.dim() != 5 or qkv.shape[2] != 3 or not qkv.is_contiguous():
    raise ValueError("expected a contiguous [batch, n, 3, heads, head_dim] tensor")
  if tiles_t is not None and not isinstance(tiles_t, TileList):
    tiles_t = tuple(tiles_t)
  return _TiledAttentionQKV.apply(qkv, tiles, tiles_t, float(scale), precision)


def _reference_options(block_q, block_k, interpret):
  """The reference's keyword arguments (pallas_attn.py:317-347) in this build's terms.

  block_q / block_k must be the tile size the lists are built with (128); num_warps, num_stages,
  bwd_num_warps and bwd_split tune the reference's Triton programs and have no counterpart (the
  kernels fix their own launch shapes), so any value is accepted; interpret=True asks for the
  CPU interpreter, which does not exist here. strict_fp32 goes to patch.resolve_precision."""
  for name, val in (("block_q", block_q), ("block_k", block_k)):
    if val is not None and val != nat.BLOCK:
      raise ValueError(f"{name}={val}: the kernels use {nat.BLOCK} x {nat.BLOCK} tiles (build the lists with "
                       f"build_tile_mask / TileList)")
  if interpret:
    raise ValueError("interpret=True: there is no CPU interpreter; the kernels run on the GPU only")


def tiled_flash_attention(q, k, v, tile_ptr, tile_kb=None, tile_bits=None, *, scale, strict_fp32=False,
                          tiles_t=None, block_q=None, block_k=None, num_warps=None, num_stages=None,
                          bwd_num_warps=None, bwd_split=None, interpret=False, precision=None):
  """q, k, v: [batch, n, heads, head_dim] float32/bfloat16 on the GPU -> [batch, n, heads, head_dim].

  The reference's signature (pallas_attn.py:317-320). ``tile_ptr`` may be a prepared TileList (then
  tile_kb and tile_bits are omitted) or the first of the three arrays of ``build_tile_mask``.
  ``tiles_t`` (TileList or array triple) is the transposed mask's list for the dK/dV kernel; it
  defaults to the forward's (symmetric masks). The products on float32 tensors follow the
  reference's rule (pallas_attn.py:336-341) with torch's float32 matmul precision in place of
  JAX's: IEEE float32 under "highest" (torch's default) or with ``strict_fp32``, bf16x3 under
  "high" / "medium" (patch.resolve_precision); ``precision`` ("native" or "bf16x3") overrides it.
  The Triton tuning arguments are accepted and have no effect (see _reference_options).
  """
  from . import patch
  del num_warps, num_stages, bwd_num_warps, bwd_split
  _reference_options(block_q, block_k, interpret)
  _check(q)
  precision = patch.resolve_precision(precision, q.dtype, strict_fp32)
  _precision(precision, q.dtype)
  tiles = tile_ptr if isinstance(tile_ptr, TileList) else (tile_ptr, tile_kb, tile_bits)
  if tiles_t is not None and not isinstance(tiles_t, TileList):
    tiles_t = tuple(tiles_t)
  return _TiledAttention.apply(q, k, v, tiles, tiles_t, float(scale), precision)
