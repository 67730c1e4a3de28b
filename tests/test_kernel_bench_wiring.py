"""The package's benchmark CLI (``lmoe.kernel_bench``, the tool the committed
profile summaries name) driven on the CPU: its layer sweeps (the reference's
latency sweep, rd.py:553-577: decode T = 1..128 and prefill T = 128..4096)
and the ragged_dot group-distribution matrix (benchmark_harness.py:100-153)
run against the recording stand-in library on a small config-5-shaped layer,
with device timing and graph capture replaced by host stand-ins, and report
one line per measurement with its FLOPs and bytes.  The numbers themselves
are the GPU's to give."""
import time

import pytest
import torch

import _stand_in
from lmoe import kernel_bench as KB
from lmoe import workloads


@pytest.fixture
def bench(monkeypatch):
  rec = _stand_in.install(monkeypatch)
  out = []

  def host_time(fn, rounds=10, calls=20, name="", graph=True):
    t0 = time.perf_counter()
    fn()
    return (time.perf_counter() - t0) * 1000

  monkeypatch.setattr(KB, "time_fn", host_time)
  monkeypatch.setattr(KB, "_capture", lambda layer, h: ((lambda: layer.forward(h)), None))
  monkeypatch.setattr(KB, "report", lambda name, ms, flops, nbytes, **kw: out.append((name, flops, nbytes, kw)))
  monkeypatch.setattr(torch.cuda, "synchronize", lambda *a, **k: None)
  monkeypatch.setattr(KB, "Config5", lambda: workloads.Config5(tokens=4096, hidden=256, latent=256, intermediate=256,
                                                               experts=128, top_k=16, local_start=16,
                                                               local_experts=16))
  return rec, out


def test_layer_sweeps_report_every_token_count(bench):
  """The stand-in writes no outputs, so the routed-row counts read back from
  the dispatch are arbitrary here; what is checked is that each line's FLOP
  count is the dense projections plus the three expert GEMMs on the routed
  rows that line reports."""
  rec, out = bench
  KB.bench_decode("cpu", 1, 1)
  KB.bench_prefill("cpu", 1, 1)
  names = [o[0] for o in out]
  assert names == [f"decode layer T={t}" for t in KB._DECODE_TOKENS] + [f"prefill layer T={t}"
                                                                           for t in KB._PREFILL_TOKENS]
  c = KB.Config5()
  for name, flops, nbytes, kw in out:
    t = kw["tokens"]
    dense = 2.0 * t * c.hidden * (c.experts + 2 * c.latent)
    assert flops == dense + 2.0 * kw["routed_rows"] * 3 * c.intermediate * c.latent, name
    assert "experts_hit" in kw and "tokens_per_s" in kw and name.endswith(f"T={t}"), name
  # decode token counts take the skinny expert GEMMs, prefill the tile kernels
  assert all(kw["skinny_expert_gemms"] == (int(n.split("=")[1]) <= 64) for n, _, _, kw in out)
  assert "lmoe_ragged_dot_mxfp4_skinny" in rec.names() and "lmoe_ragged_dot_mxfp4_rows" in rec.names()


def test_distribution_matrix_reports_every_cell(bench):
  rec, out = bench
  KB.bench_dist("cpu", 1, 1)
  assert len(out) == len(workloads.HARNESS_SHAPES) * len(workloads.HARNESS_DISTRIBUTIONS) * 2
  for name, flops, nbytes, kw in out:
    m, k, n, g = workloads.HARNESS_SHAPES[name.split()[2]]
    assert flops == 2.0 * m * k * n and nbytes > 0 and sum(kw["group_sizes"]) == m, name
  assert set(rec.names()) == {"lmoe_ragged_dot"}
