"""Every C-ABI entry point turns a null pointer for a buffer it needs into
LMOE_ERR_INVALID (or LMOE_ERR_WORKSPACE for a workspace) on the host, instead
of launching a kernel that would dereference it.  One valid call per entry
point is recorded through the Python operators, the layer and three calls
built by hand (the recording stand-in library on CPU tensors); each call is
re-issued to the real liblmoe.so first as recorded (it must pass the host
checks: LMOE_OK, or LMOE_ERR_HIP at the first HIP call on a machine without a
device), then once per pointer argument with that pointer null.  The pointers
include/lmoe.h documents as optional must still be accepted."""
import pytest
import torch

import _stand_in
from lmoe import _lib, ops
from lmoe.config import LatentMoEConfig

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
      # the one-launch path of lmoe_dispatch_local_rows takes no workspace
      small_rows = name == "lmoe_dispatch_local_rows" and (args[19] & _lib.DISPATCH_FLAG_NO_ROWS) == 0
      no_rows = name == "lmoe_dispatch_local_rows" and (args[19] & _lib.DISPATCH_FLAG_NO_ROWS) != 0
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
