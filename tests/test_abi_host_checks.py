"""The C-ABI's host-side argument checks, which stand between a bad call and
a kernel launch.  One valid call per entry point is recorded through the
Python operators, the layer and a few calls built by hand (the recording
stand-in library on CPU tensors); each call is re-issued to the real
liblmoe.so first as recorded (it must pass the host checks: LMOE_OK, or
LMOE_ERR_HIP at the first HIP call on a machine without a device), then with
one argument spoiled at a time, which the library must refuse before it
launches anything:
  * a null pointer for a buffer the call needs -> LMOE_ERR_INVALID (or
    LMOE_ERR_WORKSPACE); the pointers include/lmoe.h marks optional are
    accepted;
  * an int64 size of 2^62 -> refused (buffers beyond 2^48 elements, and no
    size product may wrap around int64);
  * an out-of-range enum (dtype, layout, mode, epilogue, activation, flags,
    zero_group) -> refused."""
import pytest
import torch

import _stand_in
from lmoe import _lib, ops

# (entry point, argument index) pairs that may be null; the stream (the last
# argument) may always be null
OPTIONAL = {
    "lmoe_router_topk": {1, 11},            # bias, scores_out
    "lmoe_router_topk_ld": {2, 12},         # bias, scores_out
    "lmoe_router_topk_proj": {2},           # bias
    "lmoe_dispatch_local": {17},            # slot_pos
    "lmoe_dispatch_local_noalloc": {17},    # slot_pos
    "lmoe_dispatch_local_small": {18},      # slot_pos
    "lmoe_dispatch_local_rows": {18},       # slot_pos (+ the workspace on the one-launch path, below)
    "lmoe_dispatch_mxfp4_skinny": {23},     # slot_pos
    "lmoe_combine_slots_rms_norm": {11},    # routed_out
}


def _collect(monkeypatch):
  rec = _stand_in.install(monkeypatch)
  bf = torch.bfloat16
  g = torch.Generator().manual_seed(0)
  R = lambda *s, dt=bf: torch.randn(*s, generator=g).to(dt)
  M, K, N, G = 64, 128, 64, 4
  gs = torch.tensor([10, 0, 20, 34], dtype=torch.int32)
  pk = torch.randint(0, 256, (G, N, K // 2), dtype=torch.uint8, generator=g)
  sc = torch.randint(120, 130, (G, N, K // 32), dtype=torch.uint8, generator=g)
  tpk = torch.zeros(G, K // 64, N, 32, dtype=torch.uint8)
  tsc = torch.zeros(G, K // 64, N, 2, dtype=torch.uint8)
  E, k, L, lat, T = 128, 8, 16, 128, 64
  idx = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)]).to(torch.int32)
  w = torch.rand(T, k, generator=g)
  mpad = ops.compute_m_padded(T, k, E, L, 2.0)
  shard = R(mpad, lat)
  slot = torch.zeros(T * k, dtype=torch.int32)
  wide = torch.randn(T, E + 256, generator=g)
  calls = []
  steps = [
      lambda: ops.ragged_dot(R(M, K), R(G, K, N), gs),
      lambda: ops.ragged_dot_gateup_situ(R(M, K), R(G, K, 2 * N), gs, 4.0, 25.0),
      lambda: ops.ragged_dot_fp8_scaled(R(M, K), R(G, K, N, dt=torch.float32).to(torch.float8_e4m3fn),
                                        torch.ones(G, K // 32, 1, N), gs),
      lambda: ops.dequantize_mxfp4(pk, sc),
      lambda: ops.mxfp4_tile_weights(pk, sc),
      lambda: ops.ragged_dot_mxfp4(R(M, K), pk, sc, gs),
      lambda: ops.ragged_dot_mxfp4(R(M, K), tpk, tsc, gs, weight_layout="tiled"),
      lambda: ops.ragged_dot_mxfp4(R(M, K), tpk, tsc, gs, weight_layout="tiled", mode="skinny"),
      lambda: ops.ragged_dot_mxfp4(R(M, K), tpk[:1], tsc[:1], torch.tensor([M], dtype=torch.int32),
                                   weight_layout="tiled", k_split=2),
      lambda: ops.ragged_dot_mxfp4(R(M, K), tpk, tsc, gs, weight_layout="tiled", mode="scaled_mfma"),
      lambda: ops.ragged_dot_mxfp4(R(M, K), tpk, tsc, gs, weight_layout="tiled", mode="scaled_mfma_fp6"),
      lambda: ops.router_topk_from_logits(R(T, E, dt=torch.float32), torch.zeros(E), k),
      lambda: ops.router_topk_project(wide[:, :E], wide[:, E:], torch.zeros(E), k),
      lambda: ops.cast_rows(torch.randn(T, 256, generator=g), bf),
      lambda: ops.dense(R(M, K), R(N, K), w_layout="nk", backend="blaslt"),
      lambda: ops.dense(R(M, K), R(N, K), w_layout="nk", backend="dense"),
      lambda: ops.dense(R(4, K), R(4096, K), w_layout="nk", backend="skinny"),
      lambda: ops.dispatch_local(idx, w, R(T, lat), 16, L, mpad, path="sort"),
      lambda: ops.dispatch_local(idx, w, R(T, lat), 16, L, mpad, path="small"),
      lambda: ops.dispatch_local(idx, w, None, 16, L, mpad, gather_rows=False, lat=lat),
      lambda: ops.dispatch_local(idx, w, R(T, lat), 16, L, mpad, skip_padding_rows=True),
      # bf16 rows through lmoe_dispatch_local_rows' counting-sort path (T*k > 8192, past the
      # one-launch kernel)
      lambda: ops.dispatch_local(idx.repeat(17, 1), w.repeat(17, 1), R(17 * T, lat), 16, L,
                                 ops.compute_m_padded(17 * T, k, E, L, 2.0), skip_padding_rows=True),
      lambda: ops.combine_slots(shard, slot, w, T, k, mode="slot_sum"),
      lambda: ops.combine_slots_rms_norm(shard, slot, w, T, k, torch.ones(lat, dtype=bf), 1e-6, mode="slot_sum",
                                         return_routed=True),
      lambda: ops._combine_shard_contribution(torch.zeros(T, lat, dtype=bf), shard,
                                              torch.zeros(mpad, dtype=torch.int32), torch.zeros(mpad)),
      lambda: ops._rms_norm(R(T, lat), torch.ones(lat, dtype=bf), 1e-6),
      lambda: ops._situ_and_mul(R(T, lat), R(T, lat), 4.0, 25.0),
      lambda: ops.add(R(T, lat), R(T, lat)),
  ]
  for step in steps:
    rec.calls.clear()
    step()
    calls += rec.calls
  import test_forward_paths as paths
  for t in (1, 512):
    layer, hidden = paths._layer(256, max(t, 16))
    rec.calls.clear()
    layer.forward(hidden[:t].contiguous())
    calls += rec.calls
  by_name = {}
  for name, args in calls:
    by_name.setdefault(name, []).append(args)
  # entry points without an operator of their own
  a = by_name["lmoe_router_topk_ld"][0]
  by_name["lmoe_router_topk"] = [(a[0],) + tuple(a[2:])]
  s = by_name["lmoe_dispatch_local_small"][0]
  by_name["lmoe_dispatch_local_rows"].append(tuple(s[:20]) + (None, 0, s[20]))  # its one-launch path, no workspace
  d = by_name["lmoe_dispatch_local"][0]
  by_name["lmoe_dispatch_local_noalloc"] = [tuple(d[:18]) + (d[20],)]
  buf = (torch.zeros(4 * 16 * 32, dtype=torch.bfloat16), torch.zeros(4 * 16 * 32, dtype=torch.bfloat16))
  by_name["lmoe_transpose"] = [(buf[0].data_ptr(), 4, 16, 32, 2, buf[1].data_ptr(), None)]
  return by_name, (shard, slot, w, idx, buf, tpk, tsc, pk, sc)


@pytest.fixture(scope="module")
def recorded():
  mp = pytest.MonkeyPatch()
  try:
    yield _collect(mp)
  finally:
    mp.undo()


def test_every_compute_entry_point_is_covered(recorded):
  by_name, _ = recorded
  sized = {n for n, (args, res) in _lib.SIGNATURES.items() if n.endswith("_size") or n.endswith("_bytes")}
  compute = set(_lib.SIGNATURES) - sized - {"lmoe_last_error", "lmoe_version", "lmoe_device_arch_ok"}
  assert compute <= set(by_name), sorted(compute - set(by_name))


def test_null_pointers_are_refused_on_the_host(recorded):
  if torch.cuda.device_count() > 0:
    return  # the recorded calls hold host pointers: replay only where nothing launches
  by_name, _ = recorded
  real = _lib.lib()
  checked = 0
  for name, variants in sorted(by_name.items()):
    argt = _lib.SIGNATURES[name][0]
    for args in variants:
      rc = getattr(real, name)(*args)
      assert rc in (_lib.OK, _lib.ERR_HIP), (name, rc, real.lmoe_last_error())
      # lmoe_dispatch_local_rows(idx, w, wdt, x, xdt, x_ld, T, k, lat, start, L, m_padded, sorted, ...,
      # flags 19, workspace 20, ...): its one-launch path (T*k <= 8192, m_padded <= 8192, L + 1 <= 1024,
      # rows wanted) takes no workspace; without rows, x and sorted_tokens may be null
      rows_call = name == "lmoe_dispatch_local_rows"
      no_rows = rows_call and (args[19] & _lib.DISPATCH_FLAG_NO_ROWS) != 0
      small_rows = (rows_call and not no_rows and args[6] * args[7] <= 8192 and args[11] <= 8192
                    and args[10] + 1 <= 1024)
      optional = OPTIONAL.get(name, set()) | ({20} if small_rows else set()) | ({3, 12} if no_rows else set())
      for i, t in enumerate(argt):
        if t is not _lib.P or not args[i] or i == len(argt) - 1:
          continue
        bad = list(args)
        bad[i] = None
        rc = getattr(real, name)(*bad)
        if i in optional:
          assert rc in (_lib.OK, _lib.ERR_HIP), (name, i, rc, real.lmoe_last_error())
        else:
          assert rc in (_lib.ERR_INVALID, _lib.ERR_WORKSPACE), (name, i, rc, real.lmoe_last_error())
        checked += 1
  assert checked > 150, checked
  rows_paths = {(a[6] * a[7] <= 8192, (a[19] & _lib.DISPATCH_FLAG_NO_ROWS) != 0)
                for a in by_name["lmoe_dispatch_local_rows"]}
  assert {(True, False), (False, False), (True, True)} <= rows_paths, rows_paths


def test_empty_batches_pass_the_host_checks(monkeypatch):
  """T = 0 (empty top-k and token tensors, whose data pointers are null) is
  a valid dispatch on both paths: every row is padding."""
  if torch.cuda.device_count() > 0:
    return
  rec = _stand_in.install(monkeypatch)
  L, lat, m_padded = 16, 64, 128
  idx = torch.empty((0, 4), dtype=torch.int32)
  w = torch.empty((0, 4), dtype=torch.float32)
  x = torch.empty((0, lat), dtype=torch.bfloat16)
  assert idx.data_ptr() == 0 and x.data_ptr() == 0
  for path in ("sort", "small"):
    ops.dispatch_local(idx, w, x, 0, L, m_padded, path=path)
  ops.dispatch_local(idx, w, None, 0, L, m_padded, gather_rows=False, lat=lat)
  real = _lib.lib()
  names = rec.names()
  assert {"lmoe_dispatch_local", "lmoe_dispatch_local_small", "lmoe_dispatch_local_rows"} <= set(names)
  for name, args in rec.calls:
    assert getattr(real, name)(*args) in (_lib.OK, _lib.ERR_HIP), (name, real.lmoe_last_error())


# int64 arguments that may be arbitrarily large: workspace sizes, and the
# skinny GEMM's bound on any group's rows (a hint; the kernel uses min(M, bound))
UNBOUNDED = {
    "lmoe_combine_scatter_add": {11},
    "lmoe_dispatch_local": {19},
    "lmoe_dispatch_local_rows": {21},
    "lmoe_ragged_dot_mxfp4_splitk": {11},
    "lmoe_ragged_dot_mxfp4_skinny": {13},
}


def test_oversized_sizes_are_refused_on_the_host(recorded):
  """Each int64 size of each recorded call set to 2^62 (one at a time): the
  call is refused on the host -- its buffers would exceed 2^48 elements, or a
  product of two sizes would wrap around int64 (e.g. T * k in the dispatch),
  which the checks must not let through."""
  if torch.cuda.device_count() > 0:
    return
  by_name, _ = recorded
  real = _lib.lib()
  checked = 0
  for name, variants in sorted(by_name.items()):
    argt = _lib.SIGNATURES[name][0]
    for args in variants:
      for i, t in enumerate(argt):
        if t is not _lib.I64 or i in UNBOUNDED.get(name, set()):
          continue
        bad = list(args)
        bad[i] = 1 << 62
        rc = getattr(real, name)(*bad)
        assert rc in (_lib.ERR_INVALID, _lib.ERR_UNSUPPORTED, _lib.ERR_WORKSPACE), (name, i, rc)
        checked += 1
  assert checked > 100, checked


def test_workspace_size_queries_refuse_what_the_entry_points_refuse():
  L = _lib.lib()
  assert L.lmoe_dispatch_workspace_size(4096, 16, 112) > 0
  for T, k, Lx in [(1 << 62, 8, 16), (8, 1 << 62, 16), (1 << 31, 2, 16), (-1, 8, 16), (64, 8, 1 << 20)]:
    assert L.lmoe_dispatch_workspace_size(T, k, Lx) == -1, (T, k, Lx)
  assert L.lmoe_combine_workspace_size(16384, 4096) > 0
  assert L.lmoe_combine_workspace_size(1 << 62, 4096) == -1 and L.lmoe_combine_workspace_size(64, -1) == -1
  assert L.lmoe_mxfp8_scale_bytes(4096, 7168) > 0 and L.lmoe_mxfp8_scale_bytes(1 << 62, 128) == -1


# int arguments read as booleans (any nonzero value is true)
BOOLEANS = {
    "lmoe_ragged_dot_gateup_situ": {11},  # round_before_act
    "lmoe_router_topk": {6},              # renorm
    "lmoe_router_topk_ld": {7},
    "lmoe_router_topk_proj": {7},
}


def test_out_of_range_enums_are_refused_on_the_host(recorded):
  """Every int argument (dtype, layout, mode, epilogue, activation, flags,
  zero_group) set to 12345 or -7 is refused, but for the boolean ones."""
  if torch.cuda.device_count() > 0:
    return
  by_name, _ = recorded
  real = _lib.lib()
  checked = 0
  for name, variants in sorted(by_name.items()):
    argt = _lib.SIGNATURES[name][0]
    for args in variants:
      for i, t in enumerate(argt):
        if t is not _lib.I32 or i in BOOLEANS.get(name, set()):
          continue
        for v in (12345, -7):
          bad = list(args)
          bad[i] = v
          rc = getattr(real, name)(*bad)
          assert rc in (_lib.ERR_INVALID, _lib.ERR_UNSUPPORTED), (name, i, v, rc)
          checked += 1
  assert checked > 100, checked


def test_last_error_is_per_thread():
  """``lmoe_last_error`` is thread-local: two host threads that each make a
  call the library refuses (null buffers) read their own message, though the
  other thread's call failed in between."""
  import threading
  real = _lib.lib()
  calls = {
      "rms_norm": lambda: real.lmoe_rms_norm(None, None, 4, 8, 1e-6, _lib.BF16, None, None),
      "add": lambda: real.lmoe_add(None, None, 8, _lib.BF16, None, None),
  }
  barrier = threading.Barrier(2, timeout=30)
  seen = {name: [] for name in calls}

  def run(name):
    for _ in range(20):
      rc = calls[name]()
      barrier.wait()  # both calls have failed before either thread reads
      seen[name].append((rc, real.lmoe_last_error().decode()))
      barrier.wait()

  threads = [threading.Thread(target=run, args=(n,)) for n in calls]
  for t in threads:
    t.start()
  for t in threads:
    t.join(60)
  for name, got in seen.items():
    assert len(got) == 20 and all(rc == _lib.ERR_INVALID and msg.startswith(name + ":") for rc, msg in got), got
