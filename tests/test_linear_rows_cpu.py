"""mha.linear_rows (the GEMM row split used by the mesh transformer without autograd) against a
plain torch linear layer: the split at a multiple of 512 rows, with and without bias. CPU,
float32 and float64. The GELU epilogue is checked on the GPU (test_transformer_gpu's inference
path), where it is hipBLASLt's tanh GELU; torch's CPU kernel for it uses another GELU form."""
import pytest
import torch
import torch.nn.functional as F

from faster_weathernext_amd.mha import ROW_QUANTUM, linear_rows


@pytest.mark.parametrize("rows", [300, ROW_QUANTUM, 2 * ROW_QUANTUM + 6])
@pytest.mark.parametrize("bias,gelu", [(False, False), (True, False)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_linear_rows_matches_linear(rows, bias, gelu, dtype):
  g = torch.Generator().manual_seed(rows)
  x = torch.randn(rows, 24, generator=g, dtype=dtype)
  w = torch.randn(40, 24, generator=g, dtype=dtype)
  b = torch.randn(40, generator=g, dtype=dtype) if bias else None
  ref = F.linear(x, w, b)
  if gelu:
    ref = F.gelu(ref, approximate="tanh")
  got = linear_rows(x, w, b, gelu=gelu)
  assert got.shape == ref.shape and got.dtype == dtype
  tol = 1e-5 if dtype == torch.float32 else 1e-12
  torch.testing.assert_close(got, ref, rtol=tol, atol=tol)


def test_linear_rows_split_rows_are_the_unsplit_rows():
  # Every row of the split result equals the same row computed on its own (float64: the GEMM
  # order cannot move a row's value beyond rounding).
  g = torch.Generator().manual_seed(1)
  x = torch.randn(ROW_QUANTUM + 3, 8, generator=g, dtype=torch.float64)
  w = torch.randn(5, 8, generator=g, dtype=torch.float64)
  got = linear_rows(x, w)
  for r in (0, ROW_QUANTUM - 1, ROW_QUANTUM, ROW_QUANTUM + 2):
    torch.testing.assert_close(got[r], x[r] @ w.t(), rtol=1e-12, atol=1e-12)
