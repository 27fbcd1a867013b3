import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "faster-weathernext_amd")
for path in (ROOT, PKG):
  if path not in sys.path:
    sys.path.insert(0, path)


def pytest_configure(config):
  config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")
  config.addinivalue_line("markers", "slow: CPU test that takes more than ~20 s")


def pytest_collection_modifyitems(config, items):
  # GPU tests run only where a GPU is visible; on a CPU-only host they are skipped, not failed.
  try:
    import torch
    have_gpu = torch.cuda.is_available()
  except Exception:  # pragma: no cover
    have_gpu = False
  if have_gpu:
    return
  skip = pytest.mark.skip(reason="no GPU visible")
  for item in items:
    if "gpu" in item.keywords:
      item.add_marker(skip)
