"""Builds libfwn_attn.so (gfx950 HIP kernels + C ABI + host mask pipeline) in-tree.

    python faster-weathernext_amd/build.py [--jobs N]

Device code is compiled with hipcc for gfx950 only; host-only C++ with g++. Packed-FP32 VALU
instructions are disabled in device code (-packed-fp32-ops). Output:
faster-weathernext_amd/faster_weathernext_amd/_lib/libfwn_attn.so
"""
import argparse
import concurrent.futures
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
LIBDIR = os.path.join(HERE, "faster_weathernext_amd", "_lib")
LIB = os.path.join(LIBDIR, "libfwn_attn.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
ARCH = "gfx950"

DEVICE_SOURCES = ["attn_bf16.hip", "attn_x3.hip", "attn_x3_dkv.hip", "attn_f32.hip", "attn_combine.hip",
                  "attn_noalloc.hip", "rows.hip"]
HOST_SOURCES = ["attn_api.cpp", "mask_host.cpp", "rows_api.cpp"]


def _run(cmd):
  proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
  # hipcc's host pass does not know the packed-fp32 target feature; that warning is expected.
  out = "\n".join(l for l in proc.stdout.splitlines() if "packed-fp32-ops" not in l)
  if proc.returncode != 0:
    raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
  return out


def build(jobs=4, verbose=False):
  """Compiles every source and links the shared library; returns its path."""
  objdir = os.path.join(HERE, "_build")
  os.makedirs(objdir, exist_ok=True)
  os.makedirs(LIBDIR, exist_ok=True)
  cmds = []
  objs = []
  for src in DEVICE_SOURCES:
    obj = os.path.join(objdir, src + ".o")
    # MFMA results in VGPRs (VGPR form): the accumulators stay where the softmax VALU code reads
    # them instead of being copied between AGPRs and VGPRs every tile.
    cmds.append([HIPCC, f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-I", INCLUDE,
                 "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                 "-mllvm", "-amdgpu-mfma-vgpr-form=1",
                 "-c", os.path.join(CSRC, src), "-o", obj])
    objs.append(obj)
  for src in HOST_SOURCES:
    obj = os.path.join(objdir, src + ".o")
    cmds.append(["g++", "-O3", "-std=c++17", "-fPIC", "-pthread", "-Wall", "-I", INCLUDE,
                 "-I", os.path.join(ROCM, "include"), "-D__HIP_PLATFORM_AMD__",
                 "-c", os.path.join(CSRC, src), "-o", obj])
    objs.append(obj)
  with concurrent.futures.ThreadPoolExecutor(max_workers=max(1, jobs)) as pool:
    for out in pool.map(_run, cmds):
      if verbose and out.strip():
        print(out)
  tmp = LIB + ".tmp"
  _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-pthread", *objs, "-o", tmp])
  os.replace(tmp, LIB)
  return LIB


def main():
  p = argparse.ArgumentParser()
  p.add_argument("--jobs", type=int, default=4)
  p.add_argument("-v", "--verbose", action="store_true")
  args = p.parse_args()
  print(build(args.jobs, args.verbose))


if __name__ == "__main__":
  sys.exit(main())
