#!/usr/bin/env python3
"""Benchmark of the block-sparse masked mesh attention on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload c3|c1|c2|c4|c5|c5bwd|c5f32|c5mha|c5stack|rows]
                    [--precision native|bf16x3] [--no-cpu]

A step is one pass of the hot path over one batch of synthetic input: for the default workload
(configuration 3 of BASELINE.json) the forward kernel plus the backward as the package's backward
runs it, on the refinement-6 mesh (40,962 nodes) with the 16-hop mask, 4 heads x 128, bf16 inputs,
fp32 accumulation. The backward is the dS exchange: delta pre-pass, dK/dV writing dS, then dQ
from dS, on one stream. With --no-ds the dQ kernel recomputes S and dP and runs on the main stream
beside dK/dV on a second stream. Inputs are resident in HBM before the timed region. The metric is effective
TFLOP/s over live 128x128 tiles (14 * D * 128^2 per live tile, batch and head for fwd + bwd;
4 * D * 128^2 for forward-only workloads). The mask build is timed separately.

Prints one JSON line (rank 0). `value` comes from K steps with nothing recorded between their
launches. A second pass of K steps records an event pair around every launch (`kernels_ms`,
`ms_per_step_with_kernel_events`). The roofline entry for the dominant kernel takes its
algorithmic FLOPs per launch over its mean HIP-event duration in a pass in which every kernel
runs alone on one stream: that event pass itself when the step is already one stream (the dS
exchange), else a third pass (with --no-ds the step runs dQ and dK/dV side by side as the package
does). And a CPU baseline: the restated reference XLA chunked
path (oracle/attention.py) on a bounded sample of query chunks of the same workload, on the cores
this process may use (os.sched_getaffinity), with the CPU model.

c5bwd and c5f32 are the reference's own attention benchmark (scripts/attn_bench.py --grad: 32-hop,
Hilbert order, 6 x 128 heads, one layer's forward + backward) in bf16 and in float32; the line
carries the reference's published RTX 5090 times for the same shape beside it. The default run
(configuration 3) also times that shape in bf16 and in float32 with bf16x3 products, 10 steps each
after the headline, under "reference_shape", and configurations 1 and 2 with their own CPU
baselines under "other_configs" (--no-extra skips both).

The CPU baseline is the median of three timed runs over one fixed subset of query chunks.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [ROOT, os.path.join(ROOT, "faster-weathernext_amd")]

METRIC = "effective attn TFLOP/s (live tiles, fwd+bwd) + sec per 0.25° 6-h step, 1 GPU"
PEAK = {"bf16": 2500.0, "f32": 157.3}  # MI355X dense MFMA TFLOP/s (vendor figures)

WORKLOADS = {
    "c1": dict(k_hop=2, heads=2, head_dim=32, batch=1, dtype="f32", backward=True, reorder=False, sigma=1.0,
               refinement=3, desc="config 1: r3 mesh (642 nodes), 2-hop, 2x32, float32, forward + backward"),
    "c2": dict(k_hop=8, heads=4, head_dim=128, batch=1, dtype="f32", backward=False, reorder=False, sigma=128 ** -0.5,
               desc="config 2: r6 mesh, 8-hop, 4x128, fp32 MFMA, forward"),
    "c3": dict(k_hop=16, heads=4, head_dim=128, batch=1, dtype="bf16", backward=True, reorder=False, sigma=1.0,
               desc="config 3: r6 mesh, 16-hop, 4x128, bf16 (fp32 accumulate), forward + backward"),
    "c4": dict(k_hop=8, heads=4, head_dim=128, batch=8, dtype="bf16", backward=True, reorder=False, sigma=1.0,
               desc="config 4: r6 mesh, 8-hop, 8 members x 4x128, bf16, forward + backward"),
    "c5": dict(k_hop=32, heads=6, head_dim=128, batch=1, dtype="bf16", backward=False, reorder=True, sigma=1.0,
               reference_ms={"fwd, TF32 dots (reference default)": 9.3, "source": "docs/validation.md:397, RTX 5090"},
               desc="WN2 mesh-transformer attention shape: r6 mesh, 32-hop, Hilbert order, 6x128, bf16, "
                    "forward (one of 24 layers)"),
    "c5bwd": dict(k_hop=32, heads=6, head_dim=128, batch=1, dtype="bf16", backward=True, reorder=True, sigma=1.0,
                  reference_ms={"fwd+bwd, TF32 dots (reference default)": 42.2, "fwd+bwd, 3xTF32 (highest)": 115.4,
                                "source": "docs/validation.md:396-397, RTX 5090"},
                  desc="the reference's attention benchmark (scripts/attn_bench.py --grad): r6 mesh, 32-hop, Hilbert "
                       "order, 6x128, bf16 (fp32 accumulate), forward + backward of one WN2 attention layer"),
    "c5f32": dict(k_hop=32, heads=6, head_dim=128, batch=1, dtype="f32", backward=True, reorder=True, sigma=1.0,
                  reference_ms={"fwd+bwd, 3xTF32 (highest)": 115.4, "fwd+bwd, IEEE fp32 dots (strict_fp32)": 797.0,
                                "source": "docs/validation.md:396-397, 405, RTX 5090"},
                  desc="the reference's attention benchmark at full precision: r6 mesh, 32-hop, Hilbert order, "
                       "6x128, float32 (fp32 MFMA), forward + backward of one WN2 attention layer"),
    "c5mha": dict(k_hop=32, heads=6, head_dim=128, batch=1, dtype="bf16", backward=True, reorder=True, sigma=1.0,
                  d_model=768,
                  desc="WN2 attention block at C5 shape: fused q/k/v projection (768 -> 3x6x128), HIP attention "
                       "read in place, mha_final projection; forward + backward, bf16, random-init weights"),
    "c5stack": dict(k_hop=32, heads=6, head_dim=128, batch=1, dtype="bf16", reorder=True, d_model=768, layers=24,
                    ffw_hidden=3072, cond_size=32,
                    desc="WN2 mesh transformer (processor) forward at C5 shape: 24 blocks (conditioned layer norms, "
                         "fused-QKV HIP attention, GELU MLP 768-3072-768), Hilbert gather/scatter fused with the "
                         "first and last layer norms; bf16, random-init weights"),
    "rows": dict(dtype="f32", channels=768, batch=1,
                 desc="Hilbert gather + first layer norm and final layer norm + affine + scatter of the node "
                      "features [1, 40962, 768] float32, once each per step (patch.py:244, 274-276, 288-292)"),
}


def parse():
  p = argparse.ArgumentParser()
  p.add_argument("--gpus", type=int, default=1)
  p.add_argument("--steps", type=int, default=20)
  # The GPU's clocks settle over the first tens of steps: at C3 the timed steps ran 1.40 ms after 3
  # warm-up steps, 1.35 after 10 and 1.335 after 30 or 100 (one box).
  p.add_argument("--warmup", type=int, default=30)
  p.add_argument("--workload", default="c3", choices=sorted(WORKLOADS))
  p.add_argument("--cpu-seconds", type=float, default=18.0,
                 help="bounded CPU-baseline length (the median of three samples of one chunk subset)")
  p.add_argument("--no-extra", action="store_true",
                 help="default workload: skip the reference-shape lines (c5bwd bf16, c5f32 bf16x3) and configs 1-2")
  p.add_argument("--no-cpu", action="store_true")
  p.add_argument("--item-tiles", type=int, default=0,
                 help="longest run of tiles per work item (0: chosen per launch by the library)")
  p.add_argument("--order", default="auto", choices=["auto", "items"],
                 help="auto: the library's choice (order tables for launches with few jobs); items: every "
                      "launch in the plain (batch, head)-major item order")
  p.add_argument("--serial-bwd", action="store_true",
                 help="run dQ and then dK/dV on one stream instead of side by side on two streams")
  p.add_argument("--no-ds", action="store_true",
                 help="the recomputing dQ kernel beside dK/dV instead of the dS exchange")
  p.add_argument("--precision", default="native", choices=["native", "bf16x3"],
                 help="float32 workloads: bf16x3 forms each product from bf16 parts (three bf16 MFMA "
                      "products) in the forward and the dS-exchange backward; with --no-ds the backward "
                      "stays IEEE fp32")
  p.add_argument("--layout", default="node", choices=["node", "head"],
                 help="storage of q, k, v, o, dO, dq, dk, dv: node-major [B, n, H, D] (the reference's "
                      "interface) or head-major [B, H, n, D] passed as strided views")
  p.add_argument("--copy-mib", type=int, default=0,
                 help="instead of the attention step, time a plain device-to-device copy of this many MiB "
                      "(the known-size kernel that scales the FETCH_SIZE / WRITE_SIZE counters)")
  return p.parse_args()


TRAFFIC_DIR = os.path.join(ROOT, "profiles")


def measured_traffic(workload, kernel, precision="native"):
  """HBM bytes per launch of `kernel` on `workload` from the committed PMC summary, if there is one.

  The summary (profiles/hbm_traffic_<kernel>_<workload>.txt, with a _bf16x3 suffix for the
  split-precision kernels) holds a line `traffic_bytes_per_launch <N>`: FETCH_SIZE + WRITE_SIZE per
  dispatch, each scaled by what the same counter reads for a copy of known size.
  """
  suffix = "" if precision == "native" else "_" + precision
  path = os.path.join(TRAFFIC_DIR, f"hbm_traffic_{kernel}_{workload}{suffix}.txt")
  if not os.path.exists(path):
    return None, None
  with open(path) as f:
    for line in f:
      parts = line.split()
      if len(parts) == 2 and parts[0] == "traffic_bytes_per_launch":
        return int(float(parts[1])), os.path.relpath(path, ROOT)
  return None, None


def copy_calibration(mib, steps, warmup):
  """Times `steps` device-to-device copies of `mib` MiB (one blit kernel each) and prints one JSON line."""
  import torch
  dev = torch.device("cuda:0")
  nbytes = mib << 20
  src = torch.ones(nbytes // 4, dtype=torch.float32, device=dev)
  dst = torch.empty_like(src)
  for _ in range(warmup):
    dst.copy_(src)
  torch.cuda.synchronize()
  start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
  start.record()
  for _ in range(steps):
    dst.copy_(src)
  stop.record()
  torch.cuda.synchronize()
  ms = start.elapsed_time(stop) / steps
  print(json.dumps({"copy_bytes_read": nbytes, "copy_bytes_written": nbytes, "steps": steps, "ms_per_copy": round(ms, 4),
                    "GB_per_s": round(2 * nbytes / (ms * 1e-3) / 1e9, 1)}), flush=True)
  return 0


def mha_block(args):
  """Times one attention block (projection, attention, final projection; forward + backward) with
  the fused in-place layout and with separate contiguous q, k, v. The metric counts attention
  FLOPs over live tiles only; the projections' GEMMs (rocBLAS/hipBLASLt) are in the step time."""
  import numpy as np
  import torch

  import faster_weathernext_amd as fwn
  cfg = WORKLOADS[args.workload]
  D, H, B, dm = cfg["head_dim"], cfg["heads"], cfg["batch"], cfg["d_model"]
  dev = torch.device("cuda:0")
  torch.cuda.set_device(dev)
  mask, lat, lon, perm = fwn.mesh_mask(6, cfg["k_hop"], reorder=cfg["reorder"])
  tiles = fwn.TileList.from_mask(mask, perm, device=dev, max_item_tiles=args.item_tiles or None)
  n, T = mask.shape[0], tiles.n_tiles
  torch.manual_seed(0)
  block = fwn.TiledMHA(dm, H, D, tiles, device=dev, dtype=torch.bfloat16)
  x = torch.randn(B, n, dm, device=dev, dtype=torch.bfloat16, requires_grad=True)
  g = torch.randn(B, n, dm, device=dev, dtype=torch.bfloat16)

  def timed(fn):
    for _ in range(args.warmup):
      fn(x).backward(g)
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(args.steps):
      fn(x).backward(g)
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / args.steps

  ms_fused = timed(block.forward)
  ms_unfused = timed(block.forward_unfused)
  flops = 14 * D * 128 * 128 * T * B * H
  value = flops / (ms_fused * 1e-3) / 1e12
  result = {
      "metric": METRIC, "value": round(value, 3), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
      "warmup": args.warmup, "ms_per_step": round(ms_fused, 4), "higher_is_better": True, "scaling": "weak",
      "vs_baseline": None, "dtype": "bf16",
      "data": "synthetic: N(0,1) node features and output gradients (torch seed 0), random-init torch weights, on "
              "a generated icosahedral mesh; no checkpoints or datasets",
      "config": {"workload": cfg["desc"], "mesh_refinement": 6, "n": n, "k_hop": cfg["k_hop"], "batch": B,
                 "heads": H, "head_dim": D, "d_model": dm, "order": "hilbert", "live_tiles": T},
      "ms_per_block_unfused": round(ms_unfused, 4),
      "fused_speedup": round(ms_unfused / ms_fused, 4),
  }
  print(json.dumps(result), flush=True)
  return 0


def row_passes(args):
  """Times the two fused row passes of a step (gather + layer norm, layer norm + affine + scatter)
  against the same work as separate torch operations, and the blocks' conditioned layer norm
  (the same pass without a permutation) against torch's layer norm, multiply and add. The metric is HBM GB/s over the passes'
  algorithmic bytes: x read once and x_out, norm_out written (gather), x read and out written
  (scatter), 5 tensors of [batch, n, channels] per step (the [batch, channels] affine and the
  permutation are negligible)."""
  import numpy as np
  import torch

  import faster_weathernext_amd as fwn
  from faster_weathernext_amd import rows
  cfg = WORKLOADS[args.workload]
  dev = torch.device("cuda:0")
  torch.cuda.set_device(dev)
  v, f, lat, lon = fwn.icosahedral_mesh(6)
  perm = torch.from_numpy(np.asarray(fwn.hilbert_order(lat, lon), np.int64)).to(dev)
  inv = torch.argsort(perm)
  B, n, C = cfg["batch"], len(lat), cfg["channels"]
  dtype = torch.float32 if cfg["dtype"] == "f32" else torch.bfloat16
  g = torch.Generator(device=dev).manual_seed(0)
  x = torch.randn(B, n, C, device=dev, generator=g).to(dtype)
  mul = 1 + 0.1 * torch.randn(B, C, device=dev, generator=g)
  add = torch.randn(B, C, device=dev, generator=g)
  stream = torch.cuda.current_stream(dev)

  def fused():
    xp, yp = rows.gather_layer_norm_forward(x, perm)
    return rows.layer_norm_scatter_forward(xp, perm, mul, add)

  def unfused():
    xp = torch.index_select(x, 1, perm)
    yp = torch.nn.functional.layer_norm(xp, (C,), eps=1e-5)
    z = torch.nn.functional.layer_norm(xp, (C,), eps=1e-5) * mul[:, None].to(dtype) + add[:, None].to(dtype)
    return torch.index_select(z, 1, inv), yp

  def timed(fn):
    for _ in range(args.warmup):
      fn()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(args.steps):
      fn()
    stop.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / args.steps

  # Per-pass durations on the launch stream (the roofline entry): each pass launched `steps` times
  # back to back between two events, so host-side call overhead overlaps the kernels.
  xp, _ = rows.gather_layer_norm_forward(x, perm)
  t_gather = timed(lambda: rows.gather_layer_norm_forward(x, perm))
  t_scatter = timed(lambda: rows.layer_norm_scatter_forward(xp, perm, mul, add))
  # The block's conditioned layer norm (the same pass without a permutation) against torch's
  # layer norm, multiply and add (2 [batch, n, channels] tensors of algorithmic traffic).
  t_affine = timed(lambda: rows.layer_norm_affine_forward(xp, mul, add))
  mul_t, add_t = mul[:, None].to(dtype), add[:, None].to(dtype)
  t_affine_torch = timed(lambda: torch.nn.functional.layer_norm(xp, (C,), eps=1e-5) * mul_t + add_t)
  ms_fused = timed(fused)
  ms_unfused = timed(unfused)
  row_bytes = B * n * C * x.element_size()
  value = 5 * row_bytes / (ms_fused * 1e-3) / 1e9
  achieved = 3 * row_bytes / (t_gather * 1e-3) / 1e9
  result = {
      "metric": "HBM GB/s of the fused Hilbert gather/scatter + layer-norm passes (algorithmic bytes), 1 GPU",
      "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
      "ms_per_step": round(ms_fused, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
      "dtype": cfg["dtype"], "data": "synthetic: N(0,1) node features (torch seed 0) on a generated icosahedral mesh",
      "config": {"workload": cfg["desc"], "mesh_refinement": 6, "n": n, "batch": B, "channels": C},
      "roofline": {"bound": "hbm", "kernel": "gather_norm", "achieved": round(achieved, 1), "peak": 8000.0,
                   "unit": "GB/s", "frac": round(achieved / 8000.0, 4),
                   "traffic": measured_traffic(args.workload, "gather_norm")[0],
                   "traffic_source": measured_traffic(args.workload, "gather_norm")[1]},
      "passes_ms": {"gather_norm": round(t_gather, 4), "norm_scatter": round(t_scatter, 4)},
      "norm_affine": {"ms": round(t_affine, 4), "gbps": round(2 * row_bytes / (t_affine * 1e-3) / 1e9, 1),
                      "ms_torch_layer_norm_mul_add": round(t_affine_torch, 4)},
      "ms_per_step_torch_separate_ops": round(ms_unfused, 4),
      "speedup_vs_torch": round(ms_unfused / ms_fused, 3),
  }
  print(json.dumps(result), flush=True)
  return 0


def mesh_stack(args):
  """Times one forward of the 24-layer mesh transformer (``transformer.MeshTransformer``) at the
  C5 shape: the part of a WN2 0.25-degree step that the attention path sits in. The GNN encoder
  and decoder and the data pipeline are not part of this build, so this is not the whole step."""
  import torch

  import faster_weathernext_amd as fwn
  cfg = WORKLOADS[args.workload]
  dev = torch.device("cuda:0")
  torch.cuda.set_device(dev)
  tiles = None
  if args.item_tiles:  # one split-K cap for every launch instead of the library's per-launch choice
    mask, _, _, perm = fwn.mesh_mask(6, cfg["k_hop"], reorder=cfg["reorder"])
    tiles = fwn.TileList.from_mask(mask, perm, device=dev, max_item_tiles=args.item_tiles)
  torch.manual_seed(0)
  t0 = time.perf_counter()
  model = fwn.MeshTransformer(6, cfg["k_hop"], cfg["layers"], cfg["d_model"], cfg["heads"], cfg["head_dim"],
                              cfg["ffw_hidden"], cfg["cond_size"], cfg["reorder"], device=dev, dtype=torch.bfloat16,
                              tiles=tiles)
  t_build = time.perf_counter() - t0
  n, B, T = model.n, cfg["batch"], model.tiles.n_tiles
  x = torch.randn(B, n, cfg["d_model"], device=dev, dtype=torch.bfloat16)
  cond = torch.randn(B, cfg["cond_size"], device=dev, dtype=torch.bfloat16)
  stream = torch.cuda.current_stream(dev)
  with torch.no_grad():
    for _ in range(args.warmup):
      model(x, cond)
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(args.steps):
      model(x, cond)
    stop.record(stream)
    torch.cuda.synchronize()
  ms = start.elapsed_time(stop) / args.steps
  attn_flops = cfg["layers"] * 4 * cfg["head_dim"] * 128 * 128 * T * B * cfg["heads"]
  result = {
      "metric": "seconds per forward of the 24-layer WN2 mesh transformer at 0.25 deg (the attention path's "
                "share of a 6-h step), 1 GPU",
      "value": round(ms * 1e-3, 5), "unit": "s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
      "ms_per_step": round(ms, 3), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
      "dtype": "bf16",
      "data": "synthetic: N(0,1) node features and conditioning (torch seed 0), random-init torch weights, on a "
              "generated icosahedral mesh; no checkpoints or datasets",
      "config": {"workload": cfg["desc"], "mesh_refinement": 6, "n": n, "k_hop": cfg["k_hop"], "batch": B,
                 "layers": cfg["layers"], "heads": cfg["heads"], "head_dim": cfg["head_dim"],
                 "d_model": cfg["d_model"], "ffw_hidden": cfg["ffw_hidden"], "live_tiles": T},
      "attention_effective_tflops": round(attn_flops / (ms * 1e-3) / 1e12, 3),
      "model_build_s": round(t_build, 2),
      "reference_step_s_rtx5090": {"full_step_tf32": 0.78, "source": "README.md:38, 87 (whole 0.25-deg step)"},
  }
  print(json.dumps(result), flush=True)
  return 0


def cpu_model():
  """The host CPU's model name (/proc/cpuinfo), or the platform's processor string."""
  try:
    with open("/proc/cpuinfo") as f:
      for line in f:
        if line.startswith("model name"):
          return line.split(":", 1)[1].strip()
  except OSError:
    pass
  import platform
  return platform.processor() or "unknown"


def cpu_baseline(cfg, q, k, v, do, mask, tiles, scale, budget_s, samples=3):
  """Times the restated reference XLA chunked path on a fixed subset of whole query chunks,
  `samples` times, with the BLAS thread pool set to the cores this process may run on; reports the
  median rate and the spread. The subset is the first query chunks, as many as the first sample
  covers in budget_s / samples seconds."""
  import numpy as np
  from threadpoolctl import threadpool_info, threadpool_limits

  from oracle import attention as A
  cores = len(os.sched_getaffinity(0))
  chunk = 512
  starts, bits, window, n_kv = A.build_chunked_mask(mask, chunk)
  D, B, H = cfg["head_dim"], cfg["batch"], cfg["heads"]

  def one(c):
    A.chunked_attention(q, k, v, starts, bits, window, n_kv, chunk, scale, chunks=[c])
    if cfg["backward"]:
      A.chunked_attention_grads(q, k, v, do, starts, bits, window, n_kv, chunk, scale, chunks=[c])

  with threadpool_limits(limits=cores):
    threads = max([t.get("num_threads", 1) for t in threadpool_info()] or [1])
    done, t0 = 0, time.perf_counter()
    while True:
      one(done)
      done += 1
      if time.perf_counter() - t0 >= budget_s / samples or done == len(starts):
        break
    first = time.perf_counter() - t0
    # A workload that finishes well inside a sample's share (configuration 1) is repeated
    # within each timed sample, so that a sample is long enough to time; one more warm pass
    # sizes the repetition.
    reps = 1
    if done == len(starts) and first < budget_s / samples / 2:
      t0 = time.perf_counter()
      for c in range(done):
        one(c)
      warm = time.perf_counter() - t0
      first += warm
      reps = max(1, int(budget_s / samples / max(warm, 1e-6)))
    times = []
    for _ in range(samples):
      t0 = time.perf_counter()
      for _ in range(reps):
        for c in range(done):
          one(c)
      times.append((time.perf_counter() - t0) / reps)
  qb_per_chunk = chunk // 128
  ptr = tiles.ptr.cpu().numpy()
  live = int(ptr[min(done * qb_per_chunk, len(ptr) - 1)] - ptr[0])
  flops = (14 if cfg["backward"] else 4) * D * 128 * 128 * live * B * H
  rates = sorted(flops / t / 1e12 for t in times)
  return {"value": float(np.median(rates)), "unit": "TFLOP/s", "cores": cores, "blas_threads": int(threads),
          "cpu_model": cpu_model(), "kind": "port", "samples": len(times),
          "spread": [round(rates[0], 5), round(rates[-1], 5)],
          "sample": f"median of {len(times)} runs over the same {done} of {len(starts)} query chunks of {chunk} "
                    f"(window {window} keys, {done / len(starts):.0%} of the workload), "
                    f"{'fwd+bwd' if cfg['backward'] else 'fwd'} float32 numpy/BLAS, "
                    + (f"{min(times):.1f}-{max(times):.1f} s each" if reps == 1 else
                       f"each run the whole workload {reps} times, {min(times) * 1e3:.1f}-{max(times) * 1e3:.1f} ms per pass"),
          "seconds": round(first + reps * sum(times), 2)}


def main():
  args = parse()
  world = int(os.environ.get("WORLD_SIZE", "1"))
  if args.gpus != 1 or world != 1:
    print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE {world}); the attention "
          "path has no multi-GPU implementation in this build.", file=sys.stderr)
    return 2
  if args.copy_mib:
    return copy_calibration(args.copy_mib, args.steps, args.warmup)
  if args.workload == "c5mha":
    return mha_block(args)
  if args.workload == "rows":
    return row_passes(args)
  if args.workload == "c5stack":
    return mesh_stack(args)
  result = attention(args)
  if result is None:
    return 2
  if args.workload == "c3" and not args.no_extra:
    result["reference_shape"] = reference_shape(args)
    result["other_configs"] = other_configs(args)
  print(json.dumps(result), flush=True)
  return 0


# The reference's own attention benchmark (scripts/attn_bench.py --grad: refinement 6, 32-hop,
# Hilbert order, 6 x 128, one layer's forward + backward), timed in the default run beside the
# configuration-3 headline: bf16, and float32 with bf16x3 products (the counterpart of the
# reference's TF32 / 3xTF32 dots), against its published RTX 5090 times.
EXTRA_STEPS, EXTRA_WARMUP = 10, 20


def reference_shape(args):
  import argparse as ap
  import torch
  out = {}
  for name, wl, prec in (("c5bwd_bf16", "c5bwd", "native"), ("c5f32_bf16x3", "c5f32", "bf16x3")):
    sub = ap.Namespace(**{**vars(args), "workload": wl, "precision": prec, "steps": EXTRA_STEPS,
                          "warmup": EXTRA_WARMUP, "no_cpu": True, "layout": "node", "item_tiles": 0})
    r = attention(sub)
    torch.cuda.empty_cache()
    out[name] = {"ms_per_layer": r["ms_per_step"], "effective_tflops": r["value"],
                 "valid_entry_tflops": r["valid_entry_tflops"], "dtype": r["dtype"], "steps": EXTRA_STEPS,
                 "warmup": EXTRA_WARMUP, "kernels_ms": r["kernels_ms"], "live_tiles": r["config"]["live_tiles"],
                 "valid_entries": r["config"]["valid_entries"],
                 "reference_rtx5090_ms": WORKLOADS[wl]["reference_ms"]}
  out["note"] = ("the reference's attention benchmark shape (scripts/attn_bench.py:23, 98-119): r6 mesh, 32-hop, "
                 "Hilbert order, 6 x 128, forward + backward of one layer; ms_per_layer against the reference's "
                 "RTX 5090 ms; valid_entry_tflops counts only the mask's valid entries (14 D per entry), which does "
                 "not depend on the tile size")
  return out


# Configurations 1 and 2 of BASELINE.json in the default run, each with the GPU step time and
# the CPU baseline of the same workload: C1 whole (two query chunks), C2 on a bounded subset.
OTHER_CPU_SECONDS = {"c1": 3.0, "c2": 9.0}


def other_configs(args):
  import argparse as ap
  import torch
  out = {}
  for wl in ("c1", "c2"):
    sub = ap.Namespace(**{**vars(args), "workload": wl, "precision": "native", "steps": EXTRA_STEPS,
                          "warmup": EXTRA_WARMUP, "no_cpu": args.no_cpu, "layout": "node", "item_tiles": 0,
                          "cpu_seconds": OTHER_CPU_SECONDS[wl]})
    r = attention(sub)
    torch.cuda.empty_cache()
    out[wl] = {"workload": r["config"]["workload"], "ms_per_step": r["ms_per_step"], "effective_tflops": r["value"],
               "dtype": r["dtype"], "steps": EXTRA_STEPS, "warmup": EXTRA_WARMUP, "kernels_ms": r["kernels_ms"],
               "live_tiles": r["config"]["live_tiles"], "roofline": {k: r["roofline"][k] for k in ("kernel", "frac")}}
    if "cpu_baseline" in r:
      out[wl]["cpu_baseline"] = r["cpu_baseline"]
  return out


def attention(args):
  """One attention workload (the forward, plus the backward as the package runs it): the result
  line as a dict, or None when the arguments do not fit the workload."""
  import numpy as np
  import torch

  import faster_weathernext_amd as fwn
  from faster_weathernext_amd import _native as nat

  cfg = WORKLOADS[args.workload]
  D, H, B = cfg["head_dim"], cfg["heads"], cfg["batch"]
  dtype = torch.bfloat16 if cfg["dtype"] == "bf16" else torch.float32
  x3 = args.precision == "bf16x3"
  if x3 and dtype != torch.float32:
    print("--precision bf16x3 applies to float32 workloads (c2, c5f32)", file=sys.stderr)
    return None
  dev = torch.device("cuda:0")
  torch.cuda.set_device(dev)

  t0 = time.perf_counter()
  refinement = cfg.get("refinement", 6)
  mask, lat, lon, perm = fwn.mesh_mask(refinement, cfg["k_hop"], reorder=cfg["reorder"])
  t_mask = time.perf_counter() - t0
  t0 = time.perf_counter()
  tiles = fwn.TileList.from_mask(mask, perm, device=dev, max_item_tiles=args.item_tiles or None)
  t_tiles = time.perf_counter() - t0
  n = mask.shape[0]
  if perm is not None:
    mask = mask[perm][:, perm]
  T = tiles.n_tiles

  # Member m draws q, k, v (N(0, sigma)) then dO (N(0, 1)) from PCG64 seed m.
  members = []
  for m in range(B):
    rng = np.random.default_rng(m)
    xs = [(cfg["sigma"] * rng.standard_normal((n, H, D))).astype(np.float32) for _ in range(3)]
    members.append(xs + [rng.standard_normal((n, H, D)).astype(np.float32)])
  host = [np.stack([mem[i] for mem in members]) for i in range(4)]
  q, k, v, do = (torch.from_numpy(x).to(dev).to(dtype) for x in host)
  if args.layout == "head":
    # [batch, n, heads, head_dim] views of head-major storage: a 32-row group of one head is one
    # contiguous run instead of 32 rows at the node stride.
    q, k, v, do = (x.permute(0, 2, 1, 3).contiguous().permute(0, 2, 1, 3) for x in (q, k, v, do))
  scale = D ** -0.5
  desc = nat.AttnDesc(B, n, H, D, nat.BF16 if dtype == torch.bfloat16 else nat.F32, scale, *q.stride()[:3])
  # bf16x3: the forward and the dS-exchange kernels take this descriptor (each splits its streamed
  # operands into the workspace first); delta and the recomputing kernels take the native one.
  fdesc = nat.AttnDesc(B, n, H, D, nat.F32, scale, *q.stride()[:3], 0, 0, 0, nat.PREC_BF16X3, 0) if x3 else desc
  out = torch.empty_like(q)
  lse = torch.empty((B, H, n), device=dev, dtype=torch.float32)
  delta = torch.empty_like(lse)
  dq, dk, dv = torch.empty_like(q), torch.empty_like(q), torch.empty_like(q)
  L = nat.lib()
  stream = torch.cuda.current_stream(dev)
  sp = stream.cuda_stream
  # The schedule of each kernel (with --order auto, its order table): the forward's, dQ's and
  # dK/dV's (the list is its own transpose); the recomputing kernels take the native descriptor.
  sched = lambda d, kernel: (tiles.struct_for_desc(d, kernel) if args.order == "auto" else
                             tiles.struct_for(B, H, kernel=kernel))
  ts, tsq, tst = sched(fdesc, "fwd"), sched(fdesc, "dq"), sched(fdesc, "kv")
  tsq_n, tst_n = sched(desc, "dq"), sched(desc, "kv")
  ws = fwn.hip_attn.workspace(fdesc, dev, tiles)
  wsp, wsn = (ws.data_ptr(), ws.numel()) if ws is not None else (None, 0)
  # dK/dV runs on a second stream beside dQ (as the package's backward does), with its own
  # workspace; the step joins the two streams at its end.
  side = torch.cuda.Stream(dev)
  ws2 = fwn.hip_attn.workspace(desc, dev, tiles)
  ws2p, ws2n = (ws2.data_ptr(), ws2.numel()) if ws2 is not None else (None, 0)

  def fwd(st):
    nat.check(L.fwn_attn_fwd_launch(fdesc, q.data_ptr(), k.data_ptr(), v.data_ptr(), ts, out.data_ptr(),
                                    lse.data_ptr(), wsp, wsn, st.cuda_stream))

  def bwd_delta(st):
    nat.check(L.fwn_attn_bwd_delta_launch(desc, out.data_ptr(), do.data_ptr(), delta.data_ptr(), st.cuda_stream))

  def bwd_dq(st):
    nat.check(L.fwn_attn_bwd_dq_launch(desc, q.data_ptr(), k.data_ptr(), v.data_ptr(), do.data_ptr(),
                                       lse.data_ptr(), delta.data_ptr(), tsq_n, dq.data_ptr(), wsp, wsn, st.cuda_stream))

  def bwd_dkv(st):
    own = st is side  # beside dQ: its own workspace
    nat.check(L.fwn_attn_bwd_dkv_launch(desc, q.data_ptr(), k.data_ptr(), v.data_ptr(), do.data_ptr(),
                                        lse.data_ptr(), delta.data_ptr(), tst_n, dk.data_ptr(), dv.data_ptr(),
                                        ws2p if own else wsp, ws2n if own else wsn, st.cuda_stream))

  # The bf16 backward's dS exchange, as the package runs it (symmetric k-hop mask: the forward
  # list is its own transpose, so one list serves both kernels).
  dmap = None
  if cfg["backward"] and not args.no_ds and fwn.hip_attn.DS_EXCHANGE:
    dmap = tiles.ds_map(tiles, fwn.hip_attn.unit_keys_for(dtype))
  if dmap is not None:
    dsbuf = torch.empty(max(dmap.ds_bytes(desc), 256), dtype=torch.uint8, device=dev)

  def bwd_dkv_ds(st):
    nat.check(L.fwn_attn_bwd_dkv_ds_launch(fdesc, q.data_ptr(), k.data_ptr(), v.data_ptr(), do.data_ptr(),
                                           lse.data_ptr(), delta.data_ptr(), tst, dmap.struct, dk.data_ptr(),
                                           dv.data_ptr(), dsbuf.data_ptr(), dsbuf.numel(), wsp, wsn, st.cuda_stream))

  def bwd_dq_ds(st):
    nat.check(L.fwn_attn_bwd_dq_ds_launch(fdesc, k.data_ptr(), dsbuf.data_ptr(), dsbuf.numel(), tsq, dmap.struct,
                                          dq.data_ptr(), wsp, wsn, st.cuda_stream))

  # (name, launch, stream it runs on). The step: with the dS exchange, every kernel in order on one
  # stream; otherwise dK/dV on the side stream after delta, beside dQ (unless --serial-bwd). The
  # solo pass: every kernel on one stream, so each has the GPU alone; the roofline entry takes the
  # dominant kernel's duration from it.
  solo = [("fwd", fwd, stream)]
  if dmap is not None:
    solo += [("delta", bwd_delta, stream), ("dkv_ds", bwd_dkv_ds, stream), ("dq_ds", bwd_dq_ds, stream)]
  elif cfg["backward"]:
    solo += [("delta", bwd_delta, stream), ("dq", bwd_dq, stream), ("dkv", bwd_dkv, stream)]
  paired = solo if args.serial_bwd or not cfg["backward"] or dmap is not None else \
      [("fwd", fwd, stream), ("delta", bwd_delta, stream), ("dkv", bwd_dkv, side), ("dq", bwd_dq, stream)]

  def step(kernels, ev=None):
    for i, (name, fn, st) in enumerate(kernels):
      if st is side:
        side.wait_stream(stream)
      if ev is not None:
        ev[i][0].record(st)
      fn(st)
      if ev is not None:
        ev[i][1].record(st)
    if any(st is side for _, _, st in kernels):
      stream.wait_stream(side)

  def timed_pass(kernels, kernel_events=True):
    """K steps between two events on the main stream and, with `kernel_events`, an event pair on
    its own stream around every launch: (ms per step, mean ms per kernel, events)."""
    events = [[[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in kernels] for _ in range(args.steps)]
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for s_ in range(args.steps):
      step(kernels, events[s_] if kernel_events else None)
    stop.record(stream)
    torch.cuda.synchronize()
    per = {name: float(np.mean([events[s_][i][0].elapsed_time(events[s_][i][1]) for s_ in range(args.steps)]))
           for i, (name, _, _) in enumerate(kernels)} if kernel_events else None
    return start.elapsed_time(stop) / args.steps, per, events

  for _ in range(args.warmup):
    step(paired)
  # Timed region 1 (the metric): K steps as the package runs them, with no event between launches.
  ms_step, _, _ = timed_pass(paired, kernel_events=False)
  # The same steps again with an event pair around every launch: the per-kernel times.
  ms_step_events, per_kernel, events = timed_pass(paired)
  pair_ms = None
  if cfg["backward"] and paired is not solo:
    # dQ and dK/dV side by side: from the end of delta (both streams start there) to the later end.
    names = [nm for nm, _, _ in paired]
    i_d, i_q, i_kv = names.index("delta"), names.index("dq"), names.index("dkv")
    pair_ms = float(np.mean([max(events[s_][i_d][1].elapsed_time(events[s_][i_q][1]),
                                 events[s_][i_d][1].elapsed_time(events[s_][i_kv][1])) for s_ in range(args.steps)]))
  # The roofline entry: K steps with every kernel alone on the GPU (the event pass when the step is
  # one stream already).
  if paired is solo:
    ms_solo, per_solo = ms_step_events, per_kernel
  else:
    for _ in range(args.warmup):
      step(solo)
    ms_solo, per_solo, _ = timed_pass(solo)

  unit_flops = D * 128 * 128 * T * B * H  # one live tile x D, all batch members and heads
  total_flops = (14 if cfg["backward"] else 4) * unit_flops
  value = total_flops / (ms_step * 1e-3) / 1e12
  # Algorithmic FLOPs per launch: forward 4*D per live entry; the backward's 10*D (FA2 count: S,
  # dP, dV, dK, dQ at 2*D each). The recomputing kernels split it as dQ 4*D (dQ + half of the S/dP
  # recompute) and dK/dV 6*D; with the dS exchange dK/dV computes S, dP, dV, dK (8*D) and dQ only
  # dQ (2*D).
  algo = {"fwd": 4 * unit_flops, "dq": 4 * unit_flops, "dkv": 6 * unit_flops, "delta": 0,
          "dkv_ds": 8 * unit_flops, "dq_ds": 2 * unit_flops}
  dominant = max((k_ for k_ in per_solo if algo.get(k_)), key=lambda k_: per_solo[k_])
  achieved = algo[dominant] / (per_solo[dominant] * 1e-3) / 1e12
  peak = PEAK[cfg["dtype"]]
  if x3 and (dominant == "fwd" or dmap is not None):
    peak = round(PEAK["bf16"] / 3, 1)  # three bf16 MFMA products per counted fp32 product
  traffic, traffic_src = measured_traffic(args.workload, dominant, args.precision)
  rate = lambda name, ms: round(algo[name] / (ms * 1e-3) / 1e12, 3)

  result = {
      "metric": METRIC, "value": round(value, 3), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
      "warmup": args.warmup, "ms_per_step": round(ms_step, 4), "higher_is_better": True, "scaling": "weak",
      "vs_baseline": None,
      "dtype": cfg["dtype"] if not x3 else ("bf16x3" if not cfg["backward"] or dmap is not None
                                            else "bf16x3 fwd, f32 bwd"),
      "data": "synthetic: N(0, sigma) q/k/v and N(0,1) dO, member m from numpy PCG64 seed m, on a generated "
              "icosahedral mesh; no weights or datasets",
      "config": {"workload": cfg["desc"], "mesh_refinement": refinement, "n": n, "k_hop": cfg["k_hop"], "batch": B,
                 "heads": H, "head_dim": D, "order": "hilbert" if cfg["reorder"] else "subdivision",
                 "sigma": cfg["sigma"], "live_tiles": T, "tile_density": round(tiles.density, 4),
                 "live_group_fraction": round(tiles.group_fraction, 4),
                 "valid_entries": int(mask.nnz),
                 "item_tiles": {kn: tiles.item_cap_for(B, H, kn) for kn in ("fwd", "dq", "kv")},
                 "order_tables": {"fwd": ts.n_work > 0, "dq": tsq.n_work > 0, "kv": tst.n_work > 0},
                 "precision": args.precision},
      "roofline": {"bound": "mfma", "kernel": dominant, "achieved": round(achieved, 3), "peak": peak,
                   "unit": "TFLOP/s", "frac": round(achieved / peak, 4), "traffic": traffic,
                   "traffic_source": traffic_src, "ms": round(per_solo[dominant], 4),
                   "work": "algorithmic FLOPs over whole live 128x128 tiles; the kernels skip 32x32 groups "
                           "without a valid element (config.live_group_fraction of them execute), so frac "
                           "can exceed 1" + ("; bf16x3: fp32-equivalent products against the bf16 MFMA "
                                             "peak / 3" if x3 and peak != PEAK["f32"] else ""),
                   "timing": ("the event pass (the metric's steps again, every kernel in order on one stream, "
                              "each alone on the GPU)" if paired is solo else
                              "solo pass: the same K steps again with every kernel on one stream (each alone on "
                              "the GPU)") + ", HIP events on that stream around each launch, split-K combine "
                                            "included"},
      "backward": None if not cfg["backward"] else (
          "dS exchange: delta, dK/dV writing dS, dQ from dS, one stream" if dmap is not None else
          "recomputing dQ kernel" + (" then dK/dV, one stream" if args.serial_bwd else
                                     " beside dK/dV on a second stream")),
      "ms_per_step_with_kernel_events": round(ms_step_events, 4),
      "kernels_ms": {k_: round(v_, 4) for k_, v_ in per_kernel.items()},
      "kernels_ms_solo": {k_: round(v_, 4) for k_, v_ in per_solo.items()},
      "kernels_tflops_solo": {k_: rate(k_, v_) for k_, v_ in per_solo.items() if algo.get(k_)},
      "ms_per_step_solo": round(ms_solo, 4),
      "valid_entry_tflops": round(value * mask.nnz / (T * 128 * 128), 3),
      "mask_build_s": round(t_mask, 3), "tile_prepare_s": round(t_tiles, 3),
      "step_s": None,
      "step_note": "the full WN2 0.25-deg step needs jax, haiku and weathernext, which this image lacks; "
                   "run --workload c5 for the attention share of a step (24 layers x forward)",
  }
  if dmap is not None:
    result["ds_exchange"] = {"units": dmap.n_units, "bytes": dmap.ds_bytes(desc),
                             "note": "dS units written by dK/dV, read by dQ: " +
                                     ("32 queries x 16 keys, bf16, 1 KB" if dmap.unit_keys == 16 else
                                      "32 queries x 32 keys, float32, 4 KB")}
  if pair_ms is not None:
    result["backward_pair"] = {
        "ms": round(pair_ms, 4), "kernels": ["dq", "dkv"], "note": "dq and dkv side by side on two streams",
        "achieved": round((algo["dq"] + algo["dkv"]) / (pair_ms * 1e-3) / 1e12, 3), "unit": "TFLOP/s",
        "frac": round((algo["dq"] + algo["dkv"]) / (pair_ms * 1e-3) / 1e12 / peak, 4)}
  if "reference_ms" in cfg:
    result["reference_rtx5090_ms"] = cfg["reference_ms"]
  if args.workload == "c5":
    result["attn_s_per_step"] = round(24 * ms_step * 1e-3, 4)
  if not args.no_cpu:
    host_np = [x.astype(np.float32) for x in host]
    result["cpu_baseline"] = cpu_baseline(cfg, *host_np, mask, tiles, scale, args.cpu_seconds)
  return result


if __name__ == "__main__":
  sys.exit(main())
