"""fwn_attn_fwd_launch_noalloc, the forward launcher that allocates nothing (split work items use
the library's static device scratch), against fwn_attn_fwd_launch with a caller workspace.

Two calls in a row share the scratch: the second, smaller call (fewer members, fewer nodes,
another mask) must not see anything of the first. Both must equal the workspace launcher bit for
bit (same kernels, same schedule), also when launched with the schedule's order table, and the
dense float64 oracle within the bars.
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


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_noalloc_forward_matches_workspace_forward(dtype):
  L = nat.lib()
  stream = torch.cuda.current_stream().cuda_stream
  rng = np.random.default_rng(70)
  for call, (b, n, h, d, cap, seed) in enumerate(((3, 900, 2, 64, 2, 71), (1, 500, 2, 64, 3, 72))):
    q, k, v = (rounded(rng.standard_normal((b, n, h, d)), dtype) for _ in range(3))
    m = random_mask(n, 0.05, seed, symmetric=True)
    tiles = fwn.TileList.from_mask(m, max_item_tiles=cap)
    assert tiles.n_split > 0  # the scratch is used
    qd, kd, vd = (dev(x, dtype) for x in (q, k, v))
    desc = nat.AttnDesc(b, n, h, d, DT[dtype], d ** -0.5, *qd.stride()[:3])
    size = ctypes.c_uint64(0)
    nat.check(L.fwn_attn_workspace_size(desc, tiles.struct, ctypes.byref(size)))
    assert 0 < size.value <= nat.SCRATCH_BYTES
    ws = torch.full((size.value,), 255, dtype=torch.uint8, device="cuda")
    want, want_lse = torch.empty_like(qd), torch.empty((b, h, n), device="cuda")
    got, got_lse = torch.full_like(qd, float("nan")), torch.full((b, h, n), float("nan"), device="cuda")
    nat.check(L.fwn_attn_fwd_launch(desc, qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), tiles.struct, want.data_ptr(),
                                    want_lse.data_ptr(), ws.data_ptr(), size.value, stream))
    nat.check(L.fwn_attn_fwd_launch_noalloc(desc, qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), tiles.struct,
                                            got.data_ptr(), got_lse.data_ptr(), stream))
    # the same forward with the order table the library launches it with: the same bits
    ordered = tiles.struct_for_desc(desc, "fwd")
    assert ordered.n_work > 0
    got2 = torch.full_like(qd, float("nan"))
    nat.check(L.fwn_attn_fwd_launch_noalloc(desc, qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), ordered,
                                            got2.data_ptr(), None, stream))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(got), host(want), err_msg=f"call {call} out")
    np.testing.assert_array_equal(host(got_lse), host(want_lse), err_msg=f"call {call} lse")
    np.testing.assert_array_equal(host(got2), host(want), err_msg=f"call {call} out, order table")
    check(host(got), A.dense_attention(q, k, v, m.toarray(), d ** -0.5), dtype, ("call", call))
