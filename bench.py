#!/usr/bin/env python3
"""LatentMoE layer benchmark on one MI355X.

One step = one full local-shard LatentMoE forward over 4096 tokens: router
logits GEMM (7168 -> 896, f32 out), down-projection (7168 -> 1024), top-16
router, local-shard dispatch (experts 0..111), fused gate/up + SiTU-GLU and
down grouped GEMMs on MXFP4 expert weights, combine, RMSNorm and the
up-projection (1024 -> 7168).  Inputs are resident in HBM before timing.

Prints ONE JSON line with the layer throughput, the roofline of the dominant
kernel (the MXFP4 gate/up grouped GEMM, timed in place with HIP events on its
stream) and the CPU baseline (the oracle's restatement of the reference
forward on a bounded token sample, timed on this host).

  python bench.py [--steps K] [--warmup W] [--rounds R] [--gpus 1] [--mxfp4-mode lds_dequant]

Timing: W warm-up steps, then K timed steps of each execution (HIP-graph
replays of the whole layer, eager launches) in R rounds whose candidate order
rotates; ms_per_step is the median over rounds of the graph replays' per-step
time (hw_session_common.py:120-175's protocol), with the per-call median
beside it.  The CPU baseline: one warm-up run, then the median of >= 5 runs.
"""

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "tokamax-tpu-kernel-lab_amd"))
sys.path.insert(0, ROOT)

METRIC = "LatentMoE layer tokens/s @1 GPU; grouped-GEMM TFLOP/s as % of MFMA peak"
HBM_PEAK_GBS = 8000.0
DEVICE = "cuda:0"  # the one GPU this benchmark measures
PEAK_TFLOPS = {"bf16": 2500.0, "mxfp4": 10100.0}


def log(msg):
  print(f"[bench] {msg}", file=sys.stderr, flush=True)


def gateup_algorithmic(c, group_sizes):
  """Algorithmic FLOPs / HBM bytes of one MXFP4 gate/up + SiTU launch:
  valid rows only, each touched expert's weights read once."""
  import numpy as np
  gs = np.asarray(group_sizes)[: c.local_experts]
  rows = int(gs.sum())
  lat, inter = c.latent, c.intermediate
  experts_hit = int((gs > 0).sum())
  w_bytes = experts_hit * 2 * inter * lat * (0.5 + 1.0 / 32)
  act_bytes = rows * lat * 2 + rows * inter * 2
  flops = 2.0 * rows * lat * 2 * inter
  return rows, experts_hit, flops, w_bytes + act_bytes


def load_traffic(name):
  path = os.path.join(ROOT, "profiles", name)
  if not os.path.exists(path):
    return None
  with open(path) as f:
    return json.load(f)


def cpu_model() -> str:
  """The host CPU as lscpu names it (its model name and, where the firmware
  reports one, the BIOS model name), with the family / model / stepping
  numbers from /proc/cpuinfo, which identify the part when a virtualised host
  hides the model number."""
  import subprocess
  names = []
  try:
    out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
    for line in out.splitlines():
      key, _, val = line.partition(":")
      if key.strip() in ("Model name", "BIOS Model name") and val.strip() and val.strip() not in names:
        names.append(val.strip())
  except (OSError, subprocess.SubprocessError):
    pass
  ids = {}
  try:
    with open("/proc/cpuinfo") as f:
      for line in f:
        key, _, val = line.partition(":")
        key = key.strip()
        if key == "model name" and val.strip() not in names:
          names.append(val.strip())
        if key in ("cpu family", "model", "stepping") and key not in ids:
          ids[key] = val.strip()
        if not line.strip() and ids:
          break
  except OSError:
    pass
  name = " / ".join(names) or "unknown"
  if ids:
    name += " (" + ", ".join(f"{k} {v}" for k, v in ids.items()) + ")"
  return name


def cpu_threads() -> tuple[int, int]:
  """(threads to use, cores in this process's affinity mask): the affinity
  mask, capped by OMP_NUM_THREADS where the host sets one (the share of a
  shared box's CPUs that one job may use)."""
  affinity = len(os.sched_getaffinity(0))
  cap = os.environ.get("OMP_NUM_THREADS", "")
  threads = min(affinity, int(cap)) if cap.isdigit() and int(cap) > 0 else affinity
  return threads, affinity


def rotated_rounds(candidates, steps, rounds, new_event, synchronize):
  """``steps`` calls of every candidate, in ``rounds`` rounds; within a round
  each candidate runs its share of calls back to back, timed by two events
  on the current stream between device synchronisations, and the candidate
  order rotates from round to round, so slow drifts of the device (clock,
  temperature) fall on every candidate alike (the protocol of
  hw_session_common.py:120-175).  ``candidates`` maps a name to a function of
  the call index; returns, per name, the per-call milliseconds of each round
  (pipelined: one event pair around the round's calls)."""
  rounds = max(1, min(rounds, steps))
  sizes = [steps // rounds + (1 if r < steps % rounds else 0) for r in range(rounds)]
  names = list(candidates)
  per = {n: [] for n in names}
  done = {n: 0 for n in names}
  for r, size in enumerate(sizes):
    for i in range(len(names)):
      name = names[(r + i) % len(names)]
      fn = candidates[name]
      synchronize()
      start, end = new_event(), new_event()
      start.record()
      for j in range(size):
        fn(done[name] + j)
      end.record()
      synchronize()
      per[name].append(start.elapsed_time(end) / size)
      done[name] += size
  return per


def per_call(fn, calls, new_event, synchronize):
  """Milliseconds of single calls, each between device synchronisations and
  timed by its own event pair."""
  out = []
  for i in range(calls):
    synchronize()
    start, end = new_event(), new_event()
    start.record()
    fn(i)
    end.record()
    synchronize()
    out.append(start.elapsed_time(end))
  return out


def oracle_inputs(layer, hidden, w, c):
  """The layer's weights as the oracle takes them: MXFP4 experts dequantised
  (bit-exact, as the reference does offline) to (L+1, in, out) f32 arrays,
  dense weights and the hidden states as f32 numpy arrays."""
  import torch

  from lmoe import ops
  E = layer.experts
  I = c.intermediate
  gu = ops.dequantize_mxfp4(E["gu_packed"], E["gu_scale"], out_dtype=torch.bfloat16)  # (L+1, 2I, lat)
  dn = ops.dequantize_mxfp4(E["down_packed"], E["down_scale"], out_dtype=torch.bfloat16)  # (L+1, lat, I)
  f = lambda t: t.float().cpu().numpy()
  gu_h, dn_h = f(gu), f(dn)
  del gu, dn
  wd = {k: f(v) for k, v in w.items()}
  return (f(hidden), wd, gu_h[:, :I, :].transpose(0, 2, 1), gu_h[:, I:, :].transpose(0, 2, 1),
          dn_h.transpose(0, 2, 1))


def cpu_baseline(inputs, c, sample_tokens, reps):
  """Oracle restatement of the reference single-shard forward on the host:
  the same weights, ``sample_tokens`` of the 4096 tokens, median of ``reps``
  runs.  Returns (baseline dict, the last run's (output, stages))."""
  from oracle import lmoe_oracle as O
  import contextlib
  threads, affinity = cpu_threads()
  try:
    from threadpoolctl import threadpool_limits
    limits = threadpool_limits(limits=threads)
  except Exception:  # noqa: BLE001
    limits = contextlib.nullcontext()
  h, wd, gate, up, down = inputs
  h = h[:sample_tokens]
  cfg = c.config()
  run = lambda: O.single_shard_forward(h, wd, gate, up, down, cfg, "bf16", c.local_start, c.local_experts,
                                       c.capacity_factor, include_shared=False)
  times = []
  with limits:
    res = run()
    for _ in range(reps):
      t0 = time.perf_counter()
      res = run()
      times.append(time.perf_counter() - t0)
  med = statistics.median(times)
  return {"value": round(sample_tokens / med, 2), "unit": "tokens/s", "cores": int(threads),
          "affinity_cores": int(affinity), "cpu_model": cpu_model(), "kind": "port",
          "sample": f"{sample_tokens} of {c.tokens} tokens through the numpy oracle's single-shard "
                    f"forward (all stages, bf16 rounding emulated), one warm-up run, then the median of "
                    f"{reps} runs ({med:.2f} s each; min {min(times):.2f}, max {max(times):.2f} s)"}, res


def parity(inputs, c, out, st, own):
  """The benchmarked forward's output against the oracle on the same tokens:
  routing on the oracle's own logits (agreement), then the oracle run on the
  device's logits and latent projection -- routing and dispatch bit-exact,
  final output max-relative error (bf16 bar 2e-2)."""
  import numpy as np
  import torch

  from oracle import lmoe_oracle as O

  def np32(t):
    t = t.detach()
    if t.dtype == torch.bfloat16:
      return t.float().cpu().numpy()
    return t.cpu().numpy()

  h, wd, gate, up, down = inputs
  cfg = c.config()
  lg, x = np32(st["router_logits"]), np32(st["x"])
  ref, rs = O.single_shard_forward(h, wd, gate, up, down, cfg, "bf16", c.local_start, c.local_experts,
                                   c.capacity_factor, include_shared=False, logits=lg, x=x)
  idx = np32(st["topk_idx"])
  out_np = np32(out)
  mr = lambda a, b: float(np.max(np.abs(a.astype(np.float64) - b)) / max(float(np.max(np.abs(b))), 1e-30))
  res = {"tolerance": 2e-2,
         "routing_bit_exact_on_device_logits": bool(np.array_equal(idx, rs["topk_idx"])
                                                    and np.array_equal(np32(st["topk_weight"]), rs["topk_weight"])),
         "dispatch_bit_exact": bool(all(np.array_equal(np32(a), b) for a, b in zip(st["dispatch"][:6], rs["dispatch"]))),
         "shard_out_max_rel": round(mr(np32(st["shard_out"]), rs["shard_out"]), 6),
         "final_max_rel": round(mr(out_np, ref), 6),
         "logits_max_rel_vs_oracle_gemm": None, "routing_identical_tokens": None}
  if own is not None:
    own_out, own_st = own
    agree = np.all(idx == own_st["topk_idx"], axis=1)
    res["logits_max_rel_vs_oracle_gemm"] = float(f"{mr(lg, own_st['router_logits']):.3e}")
    res["routing_identical_tokens"] = f"{int(agree.sum())}/{agree.size}"
    res["final_max_rel_vs_oracle_own_routing"] = round(mr(out_np[agree], own_out[agree]), 6)
  return res


def capture_layer(torch, layer, hidden):
  """Capture one layer forward as a HIP graph (torch.cuda.CUDAGraph, private
  memory pool, capture on a side stream of default priority).  Returns
  (replay, static_output), or None when a replay differs from the eager
  forward: each of three replays, with eager work in between, must match it
  bit for bit."""
  side = torch.cuda.Stream()
  side.wait_stream(torch.cuda.current_stream())
  with torch.cuda.stream(side):
    layer.forward(hidden)
  torch.cuda.current_stream().wait_stream(side)
  torch.cuda.synchronize()
  g = torch.cuda.CUDAGraph()
  with torch.cuda.graph(g):
    out = layer.forward(hidden)
  torch.cuda.synchronize()
  for _ in range(3):
    ref = layer.forward(hidden)
    torch.cuda.synchronize()
    out.zero_()
    g.replay()
    torch.cuda.synchronize()
    if not torch.equal(out, ref):
      log("graph replay differs from the eager forward: timing eager launches")
      return None
  return g.replay, out


def main():
  ap = argparse.ArgumentParser()
  ap.add_argument("--gpus", type=int, default=1)
  ap.add_argument("--steps", type=int, default=100)
  ap.add_argument("--warmup", type=int, default=20)
  ap.add_argument("--rounds", type=int, default=10, help="timing rounds the steps are split into")
  ap.add_argument("--mxfp4-mode", default="lds_dequant", choices=["lds_dequant", "scaled_mfma"])
  ap.add_argument("--cpu-sample-tokens", type=int, default=4096)
  ap.add_argument("--cpu-reps", type=int, default=5)
  ap.add_argument("--no-cpu-baseline", action="store_true")
  ap.add_argument("--eager", action="store_true",
                  help="time eager launches instead of replays of the layer captured as one HIP graph")
  args = ap.parse_args()
  if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
    print("bench.py measures one GPU only: this build has no multi-GPU path "
          "(the expert-parallel all-reduce across GPUs is not built).", file=sys.stderr)
    sys.exit(2)

  import numpy as np
  import torch

  from lmoe import _lib
  from lmoe.forward import LocalShardLatentMoE
  from lmoe.workloads import Config5, make_config5

  _lib.lib()
  dev = torch.device(DEVICE)
  c = Config5()
  log("generating config 5 inputs and MXFP4 expert weights")
  hidden, w, experts = make_config5(dev, c, "mxfp4")
  layer = LocalShardLatentMoE(c.config(), router_weight=w["router_weight"],
                              e_score_correction_bias=w["e_score_correction_bias"],
                              down_proj=w["down_proj"], up_proj=w["up_proj"], norm_scale=w["norm_scale"],
                              local_expert_start=c.local_start, local_num_experts=c.local_experts,
                              expert_format="mxfp4", experts=experts, capacity_factor=c.capacity_factor,
                              mxfp4_mode=args.mxfp4_mode)
  torch.cuda.synchronize()
  out_stages, st = layer.forward(hidden, return_stages=True)
  gs = st["dispatch"].group_sizes.cpu().numpy()
  rows, hit, flops, nbytes = gateup_algorithmic(c, gs)
  m_padded = int(gs.sum())
  log(f"routed rows R={rows} of m_padded={m_padded}, experts hit {hit}/{c.local_experts}, "
      f"group sizes min/max {gs[:c.local_experts].min()}/{gs[:c.local_experts].max()}")

  for _ in range(args.warmup):
    layer.forward(hidden)
  torch.cuda.synchronize()
  graph = None if args.eager else capture_layer(torch, layer, hidden)
  if graph is not None:
    replay = graph[0]
    for _ in range(args.warmup):
      replay()
    torch.cuda.synchronize()
  # Timed: `steps` calls of each execution (graph replays of the whole layer,
  # eager launches) in rotated rounds; the eager steps record events around
  # the two expert GEMMs (their in-layer times)
  events = [{k: (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for k in ("gateup", "down")}
            for _ in range(args.steps)]
  candidates = {"eager": lambda i: layer.forward(hidden, kernel_events=events[i])}
  if graph is not None:
    candidates = {"graph": lambda i: replay(), **candidates}
  main_exec = "graph" if graph is not None else "eager"
  new_event = lambda: torch.cuda.Event(enable_timing=True)
  t0 = time.perf_counter()
  per = rotated_rounds(candidates, args.steps, args.rounds, new_event, torch.cuda.synchronize)
  wall_s = time.perf_counter() - t0
  ms_per_step = statistics.median(per[main_exec])
  eager_ms = statistics.median(per["eager"])
  single = per_call((lambda i: replay()) if graph is not None else (lambda i: layer.forward(hidden)),
                    min(args.steps, 50), new_event, torch.cuda.synchronize)
  gateup_ms = statistics.median(e["gateup"][0].elapsed_time(e["gateup"][1]) for e in events)
  down_ms = statistics.median(e["down"][0].elapsed_time(e["down"][1]) for e in events)
  execution = ("HIP-graph replay of the whole layer (captured once; replays checked bit-exact against eager)"
               if graph is not None else "eager launches")
  timing = {"protocol": f"{len(per[main_exec])} rounds, candidates {list(candidates)} rotated per round, "
                        "each round's calls back to back between device synchronisations, HIP events; "
                        "ms_per_step = median over rounds",
            "rounds_ms_per_step": [round(v, 4) for v in per[main_exec]],
            "pipelined_mean_ms": round(statistics.mean(per[main_exec]), 4),
            "per_call_median_ms": round(statistics.median(single), 4), "per_call_calls": len(single),
            "eager_pipelined_median_ms": round(eager_ms, 4), "wall_s": round(wall_s, 3)}
  log(f"{main_exec}: {ms_per_step:.4f} ms/step (median of {len(per[main_exec])} rounds; per call "
      f"{timing['per_call_median_ms']:.4f}), eager {eager_ms:.4f} ms/step, gate/up kernel "
      f"{gateup_ms * 1000:.1f} us, down kernel {down_ms * 1000:.1f} us")
  tokens_per_s = c.tokens / (ms_per_step / 1000.0)

  # the timed forward (no stage outputs: gathered-row expert GEMM, no sorted
  # copy) against the forward whose stages the parity check below reads
  timed_equals_checked = bool(torch.equal(layer.forward(hidden), out_stages))
  log(f"timed forward == checked forward, bit for bit: {timed_equals_checked}")
  achieved = nbytes / (gateup_ms / 1000.0) / 1e9
  tflops = flops / (gateup_ms / 1000.0) / 1e12
  # the HBM rate a plain 256 MiB device copy reaches on this GPU (read +
  # write bytes / time): the practical ceiling beside the published peak
  src = torch.empty(256 << 20, dtype=torch.uint8, device=dev).fill_(1)
  dst = torch.empty_like(src)
  for _ in range(3):
    dst.copy_(src)
  ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
  ev0.record()
  for _ in range(10):
    dst.copy_(src)
  ev1.record()
  ev1.synchronize()
  copy_gbs = 2 * (256 << 20) * 10 / (ev0.elapsed_time(ev1) / 1000.0) / 1e9
  del src, dst
  # the kernel the gate/up launch ran, and the committed counter profile of
  # that kernel at this workload (HBM bytes per launch), when there is one
  if args.mxfp4_mode == "scaled_mfma":
    kernel, traffic_file = "grouped_gemm_mx_kernel (MXFP8 x MXFP4 scaled MFMA, SiTU)", None
  else:
    kernel, traffic_file = ("grouped_gemm_stream_kernel<64, 256, MXFP4, SiTU> (fused gate/up + SiTU-GLU)",
                            "traffic_cfg5_gateup_mxfp4.json")
  traffic = load_traffic(traffic_file) if traffic_file else None
  roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
              "frac": round(achieved / HBM_PEAK_GBS, 4),
              "traffic": traffic.get("bytes_per_launch") if traffic else None,
              "traffic_source": f"profiles/{traffic_file} (rocprofv3 FETCH_SIZE + WRITE_SIZE, committed)"
                                if traffic else None,
              "kernel": kernel,
              "algorithmic_bytes": int(nbytes), "algorithmic_flops": flops,
              "kernel_us": round(gateup_ms * 1000.0, 2),
              "copy_GBps": round(copy_gbs, 1), "frac_of_copy": round(achieved / copy_gbs, 4)}
  grouped = {"tflops": round(tflops, 2),
             "pct_mxfp4_peak": round(100 * tflops / PEAK_TFLOPS["mxfp4"], 2),
             "pct_bf16_peak": round(100 * tflops / PEAK_TFLOPS["bf16"], 2),
             "mfma_path": args.mxfp4_mode}

  cpu, par = None, None
  if not args.no_cpu_baseline:
    inputs = oracle_inputs(layer, hidden, w, c)
    log(f"cpu baseline on {args.cpu_sample_tokens} tokens")
    cpu, own = cpu_baseline(inputs, c, args.cpu_sample_tokens, args.cpu_reps)
    log("parity of the benchmarked forward against the oracle")
    par = parity(inputs, c, out_stages, st, own if args.cpu_sample_tokens == c.tokens else None)
    par["timed_forward_equals_checked_forward"] = timed_equals_checked
    log(f"parity: {par}")

  line = {
      "metric": METRIC, "value": round(tokens_per_s, 1), "unit": "tokens/s", "n_gpus": 1,
      "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4),
      "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
      "data": "synthetic (seeded; random-init weights, experts quantised to MXFP4)",
      "config": {"workload": "cfg5: full local-shard LatentMoE forward (BASELINE config 5)",
                 "tokens": c.tokens, "d_model": c.hidden, "latent": c.latent,
                 "intermediate": c.intermediate, "experts": c.experts, "top_k": c.top_k,
                 "local_experts": f"{c.local_start}..{c.local_start + c.local_experts - 1}",
                 "expert_weights": "mxfp4 (e2m1, e8m0 block-32)", "capacity_factor": c.capacity_factor,
                 "m_padded": m_padded, "routed_rows": rows, "router_skew": "zipf(1.2) on logits",
                 "shared_experts": 0, "parallelism": "single GPU (one expert shard)",
                 "execution": execution, "eager_ms_per_step": round(eager_ms, 4)},
      "timing": timing, "roofline": roofline, "grouped_gemm": grouped, "cpu_baseline": cpu, "parity": par,
  }
  print(json.dumps(line), flush=True)


if __name__ == "__main__":
  main()
