"""bench.py's measurement protocol, checked on the CPU with host-clock events
(the GPU run uses HIP events through the same functions): every candidate
runs exactly the requested calls, in order, split into the requested rounds
with the candidate order rotating per round; the CPU-baseline helpers report
the threads used, the affinity mask and a CPU model string."""
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
