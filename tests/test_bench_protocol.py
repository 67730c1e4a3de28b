"""bench.py's measurement protocol, checked on the CPU with host-clock events
(the GPU run uses HIP events through the same functions): every candidate
runs exactly the requested calls, in order, split into the requested rounds
with the candidate order rotating per round; the CPU-baseline helpers report
the threads used, the affinity mask and a CPU model string.  bench.main()
runs end to end against the recording stand-in library and prints one line of
the contract; parity() reports exact agreement for the oracle's own stages and
each planted difference in its own field."""
import time

import bench


class HostEvent:
  def record(self):
    self.t = time.perf_counter()

  def elapsed_time(self, other):
    return (other.t - self.t) * 1000.0


def test_rotated_rounds_runs_every_call_once_in_rotated_order():
  log = []
  cands = {"graph": lambda i: log.append(("graph", i)), "eager": lambda i: log.append(("eager", i))}
  syncs = []
  per = bench.rotated_rounds(cands, steps=23, rounds=5, new_event=HostEvent, synchronize=lambda: syncs.append(1))
  for name in cands:
    assert [i for n, i in log if n == name] == list(range(23))
    assert len(per[name]) == 5 and all(v >= 0 for v in per[name])
  # round r starts with candidate r % 2; round sizes 5, 5, 5, 4, 4
  firsts, pos = [], 0
  for size in (5, 5, 5, 4, 4):
    firsts.append(log[pos][0])
    assert {n for n, _ in log[pos:pos + size]} == {firsts[-1]}
    pos += 2 * size
  assert firsts == ["graph", "eager", "graph", "eager", "graph"]
  # a synchronisation before and after every timed block
  assert len(syncs) == 2 * 5 * 2


def test_rounds_are_capped_by_steps_and_timing_is_per_call():
  calls = []
  per = bench.rotated_rounds({"graph": lambda i: (calls.append(i), time.sleep(0.002))}, steps=3, rounds=10,
                             new_event=HostEvent, synchronize=lambda: None)
  assert calls == [0, 1, 2] and len(per["graph"]) == 3
  assert all(1.5 <= v <= 50 for v in per["graph"]), per
  single = bench.per_call(lambda i: time.sleep(0.001), 4, HostEvent, lambda: None)
  assert len(single) == 4 and all(0.5 <= v <= 50 for v in single)


def test_cpu_threads_and_model():
  threads, affinity = bench.cpu_threads()
  assert 1 <= threads <= affinity
  name = bench.cpu_model()
  assert name and name != "unknown"


class _TorchEvent(HostEvent):
  """torch.cuda.Event's interface over the host clock."""

  def __init__(self, enable_timing=False):
    self.t = None

  def synchronize(self):
    pass


def test_main_prints_one_line_of_the_contract(monkeypatch, capsys):
  """bench.main() end to end on the CPU -- the layer's host logic against the
  recording stand-in library, host-clock events, a small config-5 shape,
  eager launches (graph capture needs a device) -- prints exactly one JSON
  line with the contract's keys, ms_per_step the median of the timed rounds
  and value the tokens of one step over it."""
  import functools
  import json
  import statistics
  import sys

  import torch

  import _stand_in
  from lmoe import workloads
  rec = _stand_in.install(monkeypatch)
  monkeypatch.setattr(torch.cuda, "Event", _TorchEvent)
  monkeypatch.setattr(torch.cuda, "synchronize", lambda *a: None)
  monkeypatch.setattr(bench, "DEVICE", "cpu")
  small = functools.partial(workloads.Config5, tokens=512, hidden=256, latent=256, intermediate=256, experts=128,
                            top_k=16, local_start=16, local_experts=16)
  monkeypatch.setattr(workloads, "Config5", small)
  monkeypatch.setattr(sys, "argv", ["bench.py", "--eager", "--no-cpu-baseline", "--steps", "7", "--rounds", "3",
                                    "--warmup", "2"])
  bench.main()
  lines = [l for l in capsys.readouterr().out.splitlines() if l.strip()]
  assert len(lines) == 1
  line = json.loads(lines[0])
  for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better", "scaling",
              "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline", "timing"):
    assert key in line, key
  assert line["n_gpus"] == 1 and line["steps"] == 7 and line["warmup"] == 2 and line["higher_is_better"] is True
  assert line["dtype"] == "bf16" and line["unit"] == "tokens/s" and line["vs_baseline"] is None
  assert line["config"]["workload"].startswith("cfg5") and line["config"]["tokens"] == 512
  assert line["config"]["execution"] == "eager launches"
  rounds = line["timing"]["rounds_ms_per_step"]
  assert len(rounds) == 3
  assert abs(line["ms_per_step"] - statistics.median(rounds)) <= 1e-4
  assert abs(line["value"] - 512 / (line["ms_per_step"] / 1000)) <= 1e-3 * line["value"] + 0.1
  roof = line["roofline"]
  assert set(("bound", "achieved", "peak", "unit", "frac", "traffic")) <= set(roof)
  assert roof["bound"] == "hbm" and roof["peak"] == 8000.0 and roof["unit"] == "GB/s"
  # frac and achieved are rounded to 4 and 1 decimals (the stand-in's group
  # sizes are whatever the output allocation held, so the numbers themselves
  # mean nothing here)
  assert abs(roof["frac"] - roof["achieved"] / roof["peak"]) <= 1e-4 + 1e-6 * abs(roof["frac"])
  assert line["cpu_baseline"] is None and line["parity"] is None
  # the stage-returning forward, 2 warm-up steps, 7 timed steps, 7 single
  # timed calls and the equality check: 18 forwards, each with two expert GEMM
  # launches
  gemms = rec.names().count("lmoe_ragged_dot_mxfp4_rows") + rec.names().count("lmoe_ragged_dot_mxfp4")
  assert gemms == 2 * (1 + 2 + 7 + 7 + 1)
  assert line["timing"]["per_call_calls"] == 7


def test_main_refuses_more_than_one_gpu(monkeypatch, capsys):
  import sys

  import pytest
  monkeypatch.setattr(sys, "argv", ["bench.py", "--gpus", "8"])
  with pytest.raises(SystemExit) as e:
    bench.main()
  assert e.value.code == 2
  assert "one GPU only" in capsys.readouterr().err


def _oracle_inputs_cpu(c):
  """bench.oracle_inputs on the CPU: the experts dequantised by the oracle
  (the benchmark dequantises them on the device, bit-exact)."""
  from lmoe.workloads import make_config5
  from oracle import lmoe_oracle as O
  hidden, w, ex = make_config5("cpu", c, "mxfp4")
  gu = O.dequantize_mxfp4(ex["gu_packed"].numpy(), ex["gu_scale"].numpy())
  dn = O.dequantize_mxfp4(ex["down_packed"].numpy(), ex["down_scale"].numpy())
  f = lambda t: t.float().numpy()
  I = c.intermediate
  return (f(hidden), {k: f(v) for k, v in w.items()}, gu[:, :I, :].transpose(0, 2, 1),
          gu[:, I:, :].transpose(0, 2, 1), dn.transpose(0, 2, 1))


def test_cpu_baseline_and_parity_with_the_oracle_as_device():
  """cpu_baseline reports its runs, threads and sample; parity() given the
  oracle's own stages as the device's reports exact agreement, and reports
  each planted difference (a routed expert, a shard-output row, the final
  output) in its own field."""
  import numpy as np
  import torch

  from lmoe.workloads import Config5
  c = Config5(tokens=128, hidden=256, latent=256, intermediate=256, experts=128, top_k=16, local_start=16,
              local_experts=16)
  inputs = _oracle_inputs_cpu(c)
  cpu, own = bench.cpu_baseline(inputs, c, c.tokens, reps=2)
  assert cpu["kind"] == "port" and cpu["unit"] == "tokens/s" and cpu["value"] > 0
  assert 1 <= cpu["cores"] <= cpu["affinity_cores"] and "median of 2 runs" in cpu["sample"]
  own_out, own_st = own
  t = lambda a: torch.from_numpy(np.ascontiguousarray(a))
  st = {k: t(own_st[k]) for k in ("x", "router_logits", "topk_idx", "topk_weight", "shard_out")}
  st["dispatch"] = tuple(t(a) for a in own_st["dispatch"])
  assert int(own_st["dispatch"].group_sizes[:c.local_experts].sum()) > 0
  par = bench.parity(inputs, c, t(own_out), st, own)
  assert par["routing_bit_exact_on_device_logits"] and par["dispatch_bit_exact"]
  assert par["final_max_rel"] == 0.0 and par["shard_out_max_rel"] == 0.0
  assert par["routing_identical_tokens"] == f"{c.tokens}/{c.tokens}" and par["logits_max_rel_vs_oracle_gemm"] == 0.0
  # planted differences
  bad = dict(st, shard_out=st["shard_out"].clone())
  bad["shard_out"][0] *= 1.5
  p = bench.parity(inputs, c, t(own_out), bad, own)
  assert p["shard_out_max_rel"] > 0 and p["final_max_rel"] == 0.0
  out = t(own_out).clone()
  out[3] += out.abs().max()
  assert bench.parity(inputs, c, out, st, own)["final_max_rel"] > 2e-2
  bad = dict(st, topk_idx=st["topk_idx"].clone())
  bad["topk_idx"][0, 0] = (bad["topk_idx"][0, 0] + 1) % c.experts
  p = bench.parity(inputs, c, t(own_out), bad, own)
  assert not p["routing_bit_exact_on_device_logits"] and p["routing_identical_tokens"] == f"{c.tokens - 1}/{c.tokens}"
