"""The C-ABI sees pointers and sizes only, so nothing in the library can tell
that a buffer is shorter than its sizes say: that guarantee is the Python
operators'.  Here every pointer the operators hand the library is recorded
with the bytes its tensor holds from that address on, and each call's sizes
are turned into the bytes every buffer must hold (the buffer shapes
include/lmoe.h documents); a buffer shorter than that would be read or
written past its end on the device.  Checked for one call of every entry
point, for whole layer forwards in each of their paths, and for operator
calls on arbitrary (mostly inconsistent) shapes, which must either raise or
pass buffers that hold what the sizes say."""
import itertools

import pytest
import torch

import _stand_in
from lmoe import _lib, ops

SITU = _lib.EPI_SITU


def _es(dt):
  return {_lib.F32: 4, _lib.BF16: 2}.get(dt, 0)


def _rows(n, ld, width, es):
  """Bytes spanned by n rows of `width` elements, ld elements apart."""
  return 0 if n <= 0 or width <= 0 else ((n - 1) * ld + width) * es


def _scale_bytes(m, k):
  return (k // 128) * (-(-m // 4) * 4) * 4


def _w(n, epi):
  return n // 2 if epi == SITU else n


def _mx(a, wp, ws, gs, g, n, k):
  return {wp: g * n * k // 2, ws: g * n * k // 32, gs: g * 4}


# entry point -> {pointer argument index: bytes it must hold}, from the sizes
SPECS = {
    "lmoe_ragged_dot": lambda a: {0: a[5] * a[6] * _es(a[1]), 2: a[8] * a[6] * a[7] * _es(a[1]), 4: a[8] * 4,
                                  10: a[5] * a[7] * _es(a[11])},
    "lmoe_ragged_dot_gateup_situ": lambda a: {0: a[4] * a[5] * 2, 1: a[7] * a[5] * 2 * a[6] * 2, 3: a[7] * 4,
                                              12: a[4] * a[6] * 2},
    "lmoe_ragged_dot_fp8_scaled": lambda a: {0: a[5] * a[6] * 2, 1: a[8] * a[6] * a[7],
                                             2: a[8] * (a[6] // a[3] if a[3] > 0 else 0) * a[7] * 4, 4: a[8] * 4,
                                             13: a[5] * _w(a[7], a[10]) * 2},
    "lmoe_mxfp4_dequant": lambda a: {0: a[2] * a[3] * a[4] // 2, 1: a[2] * a[3] * (a[4] // a[5] if a[5] > 0 else 0),
                                     6: a[2] * a[3] * a[4] * _es(a[7])},
    "lmoe_ragged_dot_mxfp4": lambda a: {0: a[4] * a[5] * 2, **_mx(a, 1, 2, 3, a[7], a[6], a[5]),
                                        13: a[4] * _w(a[6], a[10]) * 2},
    "lmoe_ragged_dot_mxfp4_rows": lambda a: {0: a[1] * a[7] * 2, 2: a[6] * 4, **_mx(a, 3, 4, 5, a[9], a[8], a[7]),
                                             15: a[6] * _w(a[8], a[12]) * 2},
    "lmoe_ragged_dot_mxfp4_splitk": lambda a: {0: a[4] * a[5] * 2, **_mx(a, 1, 2, 3, a[7], a[6], a[5]),
                                               10: a[9] * a[4] * a[6] * 4 if a[9] > 1 else 0,
                                               15: a[4] * _w(a[6], a[12]) * 2},
    "lmoe_ragged_dot_mxfp4_skinny": lambda a: {0: a[4] * a[5] * 2, **_mx(a, 1, 2, 3, a[7], a[6], a[5]),
                                               14: a[4] * _w(a[6], a[10]) * 2},
    "lmoe_dispatch_mxfp4_skinny": lambda a: {
        0: a[5] * a[6] * 4, 1: a[5] * a[6] * _es(a[2]), 3: _rows(a[5], a[4], a[12], 2),
        **_mx(a, 10, 11, 18, a[8] + 1, a[13], a[12]), 19: a[9], 20: a[8] * 4, 21: a[9] * 4,
        22: a[9] * _es(a[2]), 23: a[5] * a[6] * 4, 24: a[9] * _w(a[13], a[14]) * 2},
    "lmoe_mxfp4_tile": lambda a: {0: a[2] * a[3] * a[4] // 2, 1: a[2] * a[3] * a[4] // 32,
                                  5: a[2] * a[3] * a[4] // 2, 6: a[2] * a[3] * a[4] // 32},
    "lmoe_quantize_mxfp8": lambda a: {0: a[2] * a[3] * _es(a[1]), 4: a[2] * a[3], 5: _scale_bytes(a[2], a[3])},
    "lmoe_quantize_mxfp6": lambda a: {0: a[2] * a[3] * _es(a[1]), 4: a[2] * a[3] * 3 // 4,
                                      5: _scale_bytes(a[2], a[3])},
    "lmoe_ragged_dot_mxfp6_mxfp4": lambda a: {0: a[5] * a[6] * 3 // 4, 1: _scale_bytes(a[5], a[6]),
                                              **_mx(a, 2, 3, 4, a[8], a[7], a[6]), 10: a[5] * a[7] * _es(a[11])},
    "lmoe_ragged_dot_mxfp8_mxfp4": lambda a: {0: a[5] * a[6], 1: _scale_bytes(a[5], a[6]),
                                              **_mx(a, 2, 3, 4, a[8], a[7], a[6]),
                                              13: a[5] * _w(a[7], a[10]) * (2 if a[10] == SITU else _es(a[14]))},
    "lmoe_router_topk": lambda a: {0: a[2] * a[3] * 4, 1: a[3] * 4, 9: a[2] * a[4] * 4, 10: a[2] * a[4] * _es(a[8]),
                                   11: a[2] * a[3] * 4},
    "lmoe_router_topk_ld": lambda a: {0: _rows(a[3], a[1], a[4], 4), 2: a[4] * 4, 10: a[3] * a[5] * 4,
                                      11: a[3] * a[5] * _es(a[9]), 12: a[3] * a[4] * 4},
    "lmoe_router_topk_proj": lambda a: {0: _rows(a[3], a[1], a[4], 4), 2: a[4] * 4, 10: a[3] * a[5] * 4,
                                        11: a[3] * a[5] * _es(a[9]), 12: _rows(a[3], a[13], a[14], 4),
                                        15: a[3] * a[14] * 2},
    "lmoe_dispatch_local": lambda a: {
        0: a[5] * a[6] * 4, 1: a[5] * a[6] * _es(a[2]), 3: a[5] * a[7] * _es(a[4]), 11: a[10] * a[7] * _es(a[4]),
        12: (a[9] + 1) * 4, 13: a[10], 14: a[9] * 4, 15: a[10] * 4, 16: a[10] * _es(a[2]), 17: a[5] * a[6] * 4,
        18: a[19]},
    "lmoe_dispatch_local_small": lambda a: {
        0: a[6] * a[7] * 4, 1: a[6] * a[7] * _es(a[2]), 3: _rows(a[6], a[5], a[8], _es(a[4])),
        12: a[11] * a[8] * 2, 13: (a[10] + 1) * 4, 14: a[11], 15: a[10] * 4, 16: a[11] * 4,
        17: a[11] * _es(a[2]), 18: a[6] * a[7] * 4},
}
SPECS["lmoe_dispatch_local_noalloc"] = lambda a: {i: v for i, v in SPECS["lmoe_dispatch_local"](a).items()
                                                  if i != 18}
SPECS["lmoe_dispatch_local_rows"] = lambda a: {**SPECS["lmoe_dispatch_local_small"](a), 20: a[21]}
SPECS.update({
    "lmoe_combine_scatter_add": lambda a: {0: a[5] * a[6] * _es(a[1]), 2: a[5] * 4, 3: a[5] * _es(a[4]),
                                           8: a[7] * a[6] * _es(a[9]), 10: a[11]},
    # shard_out rows are read at the slot positions the dispatch wrote (the
    # header asks for at least one row); scatter-mode weights likewise
    "lmoe_combine_slots": lambda a: {0: a[7] * _es(a[1]) if a[5] > 0 else 0, 2: a[5] * a[6] * 4,
                                     3: a[5] * a[6] * _es(a[4]) if a[8] == _lib.COMBINE_SLOT_SUM else 0,
                                     9: a[5] * a[7] * _es(a[10])},
    "lmoe_combine_slots_rms_norm": lambda a: {0: a[7] * _es(a[1]) if a[5] > 0 else 0, 2: a[5] * a[6] * 4,
                                              3: a[5] * a[6] * _es(a[4]) if a[8] == _lib.COMBINE_SLOT_SUM else 0,
                                              9: a[7] * _es(a[13]), 11: a[5] * a[7] * _es(a[13]),
                                              12: a[5] * a[7] * _es(a[13])},
    "lmoe_rms_norm": lambda a: {0: a[2] * a[3] * _es(a[5]), 1: a[3] * _es(a[5]), 6: a[2] * a[3] * _es(a[5])},
    "lmoe_dense_blaslt": lambda a: {0: a[4] * a[5] * _es(a[1]), 2: a[6] * a[5] * _es(a[3]),
                                    7: a[4] * a[6] * _es(a[8])},
    "lmoe_dense": lambda a: {0: a[2] * a[3] * 2, 1: a[4] * a[3] * 2, 5: a[2] * a[4] * _es(a[6])},
    "lmoe_situ_and_mul": lambda a: {0: a[2] * _es(a[5]), 1: a[2] * _es(a[5]), 6: a[2] * _es(a[5])},
    "lmoe_add": lambda a: {0: a[2] * _es(a[3]), 1: a[2] * _es(a[3]), 4: a[2] * _es(a[3])},
    "lmoe_cast_rows": lambda a: {0: _rows(a[2], a[4], a[3], _es(a[1])), 5: a[2] * a[3] * _es(a[6])},
    "lmoe_transpose": lambda a: {0: a[1] * a[2] * a[3] * a[4], 5: a[1] * a[2] * a[3] * a[4]},
})
SPECS["lmoe_dense_skinny"] = SPECS["lmoe_dense"]


class ExtentLog:
  """Installs the recording stand-in and notes, for every library call, the
  bytes each pointer argument's tensor holds from that address on."""

  def __init__(self, monkeypatch):
    self.calls = []
    pending = {}
    self._pending = pending
    orig_ga = _stand_in.RecordingLib.__getattr__
    log = self

    def p(t):
      if t is None:
        return None
      avail = t.untyped_storage().nbytes() - t.storage_offset() * t.element_size()
      ptr = t.data_ptr()
      pending[ptr] = min(pending.get(ptr, avail), avail)
      return ptr

    def ga(lib, name):
      f = orig_ga(lib, name)
      if name.endswith("workspace_size"):
        return f

      def entry(*args):
        log.calls.append((name, args, dict(pending)))
        pending.clear()
        return f(*args)
      return entry

    monkeypatch.setattr(_stand_in.RecordingLib, "__getattr__", ga)
    self.rec = _stand_in.install(monkeypatch)
    monkeypatch.setattr(ops, "_p", p)

  def clear(self):
    self.calls.clear()
    self._pending.clear()


def check_extents(calls):
  """Every non-null pointer argument holds the bytes its call's sizes ask for;
  returns the number of buffers checked."""
  checked = 0
  for name, args, avail in calls:
    assert name in SPECS, f"no extent rule for {name}"
    need = SPECS[name](args)
    pointer_args = [i for i, t in enumerate(_lib.SIGNATURES[name][0][:-1]) if t is _lib.P]
    assert set(need) == set(pointer_args), (name, sorted(set(pointer_args) ^ set(need)))
    for i, req in need.items():
      ptr = args[i]
      if ptr is None or req <= 0:
        continue
      assert ptr in avail, (name, i)
      assert req <= avail[ptr], f"{name}: argument {i} needs {req} bytes, its tensor holds {avail[ptr]}"
      checked += 1
  return checked


def test_every_entry_point_has_an_extent_rule():
  compute = {n for n, (args, ret) in _lib.SIGNATURES.items() if _lib.P in args}
  assert compute == set(SPECS), sorted(compute ^ set(SPECS))


def test_one_call_of_every_operator(monkeypatch):
  import test_abi_host_checks as H
  log = ExtentLog(monkeypatch)
  H._collect(monkeypatch)
  names = {n for n, _, _ in log.calls}
  assert len(names) >= 29, sorted(names)
  assert check_extents(log.calls) > 150


LAYER_CASES = [
    # latent, tokens, mxfp4 mode, return stages
    (256, 1, "lds_dequant", False), (256, 16, "lds_dequant", True), (256, 64, "lds_dequant", False),
    (256, 512, "lds_dequant", False), (256, 512, "lds_dequant", True), (256, 512, "scaled_mfma", False),
    (1024, 1, "lds_dequant", False), (1024, 200, "lds_dequant", False), (2048, 1, "lds_dequant", False),
    (2048, 512, "lds_dequant", False), (2048, 512, "lds_dequant", True),
]


@pytest.mark.parametrize("lat,tokens,mode,stages", LAYER_CASES)
def test_layer_forwards(monkeypatch, lat, tokens, mode, stages):
  import test_forward_paths as paths
  log = ExtentLog(monkeypatch)
  layer, hidden = paths._layer(lat, max(tokens, 16), mode=mode)
  log.clear()
  layer.forward(hidden[:tokens].contiguous(), return_stages=stages)
  assert len(log.calls) >= 5
  assert check_extents(log.calls) > 20


def test_a_short_buffer_is_caught():
  """The check itself: a recorded ragged_dot whose output tensor is one row
  short of M fails."""
  M, K, N, G = 8, 16, 8, 2
  args = (1, _lib.BF16, 2, _lib.RHS_GKN, 3, M, K, N, G, -1, 4, _lib.BF16, None)
  avail = {1: M * K * 2, 2: G * K * N * 2, 3: G * 4, 4: (M - 1) * N * 2}
  with pytest.raises(AssertionError, match="argument 10"):
    check_extents([("lmoe_ragged_dot", args, avail)])
  avail[4] = M * N * 2
  assert check_extents([("lmoe_ragged_dot", args, avail)]) == 4


# ---- operator calls on arbitrary shapes ---------------------------------------------
from hypothesis import HealthCheck, given, settings  # noqa: E402
from hypothesis import strategies as st  # noqa: E402

DIMS = [0, 1, 2, 3, 8, 16, 32, 64, 128, 256]
bf, f32, u8, i32 = torch.bfloat16, torch.float32, torch.uint8, torch.int32


def _t(shape, dtype):
  return torch.zeros(tuple(max(int(s), 0) for s in shape), dtype=dtype)


class _Draw:
  def __init__(self, data):
    self.data = data

  def dim(self):
    return self.data.draw(st.sampled_from(DIMS))

  def near(self, v):
    """v most of the time, else one off, zero or another size."""
    if self.data.draw(st.integers(0, 5)):
      return v
    return self.pick([max(v - 1, 0), v + 1, 0, self.dim()])

  def pick(self, options):
    return self.data.draw(st.sampled_from(options))


def _ragged_dot(d):
  m, k, n, g = d.dim(), d.pick([8, 16, 64, 128]), d.pick([8, 16, 64]), d.pick([1, 2, 3, 4])
  dt = d.pick([bf, f32])
  layout = d.pick(["gkn", "gnk"])
  rhs = (d.near(g), d.near(k), d.near(n)) if layout == "gkn" else (d.near(g), d.near(n), d.near(k))
  ops.ragged_dot(_t((d.near(m), d.near(k)), dt), _t(rhs, d.pick([dt, dt, bf, f32])), _t((d.near(g),), i32),
                 preferred_element_type=d.pick([None, f32]), rhs_layout=layout, zero_group=d.pick([-1, 0, g - 1, g]))


def _gateup(d):
  m, k, i, g = d.dim(), d.pick([8, 16, 64]), d.pick([8, 16, 32]), d.pick([1, 2, 4])
  layout = d.pick(["gkn", "gnk"])
  rhs = (d.near(g), d.near(k), d.near(2 * i)) if layout == "gkn" else (d.near(g), d.near(2 * i), d.near(k))
  ops.ragged_dot_gateup_situ(_t((d.near(m), d.near(k)), bf), _t(rhs, bf), _t((d.near(g),), i32), 4.0, 25.0,
                             rhs_layout=layout, zero_group=d.pick([-1, g - 1]))


def _fp8(d):
  m, k, n, g = d.dim(), d.pick([32, 64, 128]), d.pick([8, 16, 64]), d.pick([1, 2, 4])
  bs = d.pick([k, 32])
  ops.ragged_dot_fp8_scaled(_t((d.near(m), d.near(k)), bf), _t((d.near(g), d.near(k), d.near(n)), torch.float8_e4m3fn),
                            _t((d.near(g), d.near(k // bs), 1, d.near(n)), f32), _t((d.near(g),), i32),
                            fuse_gateup_activation=d.pick([None, "situ:4:25"]))


def _mx_weights(d, g, n, k, tiled):
  if tiled:
    return (_t((d.near(g), d.near(k // 64), d.near(n), d.near(32)), u8),
            _t((d.near(g), d.near(k // 64), d.near(n), d.near(2)), u8))
  return _t((d.near(g), d.near(n), d.near(k // 2)), u8), _t((d.near(g), d.near(n), d.near(k // 32)), u8)


def _mxfp4(d):
  m, k, n, g = d.dim(), d.pick([64, 128, 256]), d.pick([16, 32, 64]), d.pick([1, 2, 3])
  tiled = d.pick([True, True, False])
  # mostly the combinations the operator takes, some it refuses
  mode = d.pick(["lds_dequant", "lds_dequant", "skinny", "scaled_mfma", "scaled_mfma_fp6"] if tiled else
                ["lds_dequant", "lds_dequant", "lds_dequant", "skinny"])
  wp, ws = _mx_weights(d, g, n, k, tiled)
  gather = d.pick([False, True] if tiled and mode == "lds_dequant" else [False, False, False, True])
  row_index = _t((d.near(m),), i32) if gather else None
  lhs = _t((d.near(m if row_index is None else d.dim()), d.near(k)), bf)
  ops.ragged_dot_mxfp4(lhs, wp, ws, _t((d.near(g),), i32),
                       fuse_gateup_activation=d.pick([None, "situ:4:25"] if mode != "scaled_mfma_fp6" else
                                                     [None, None, None, "situ:4:25"]),
                       mode=mode,
                       zero_group=d.pick([-1, g - 1]), weight_layout="tiled" if tiled else "checkpoint",
                       skip_zero_group_rows=d.pick([False, True]), max_group_rows=d.pick([0, 1, 16]),
                       k_split=d.pick([None, 1, 2, 3]), lhs_row_index=row_index)


def _mx_prep(d):
  k, n, g = d.pick([64, 128, 256]), d.pick([8, 16, 64]), d.pick([1, 2])
  wp, ws = _mx_weights(d, g, n, k, False)
  if d.pick([True, False]):
    ops.dequantize_mxfp4(wp, ws, out_dtype=d.pick([f32, bf]))
  else:
    ops.mxfp4_tile_weights(wp, ws)


def _scaled(d):
  m, k, n, g = d.dim(), d.pick([128, 256]), d.pick([16, 32, 64]), d.pick([1, 2])
  fp6 = d.pick([True, False])
  if d.pick([True, False]):
    (ops.quantize_mxfp6 if fp6 else ops.quantize_mxfp8)(_t((d.near(m), d.near(k)), d.pick([bf, f32])))
    return
  q = _t((d.near(m), d.near(k * 3 // 4 if fp6 else k)), u8)
  qs = _t((d.near(k // 128), d.near(-(-m // 4) * 4), d.near(4)), u8)
  wp, ws = _mx_weights(d, g, n, k, True)
  if fp6:
    ops.ragged_dot_mxfp6_mxfp4(q, qs, wp, ws, _t((d.near(g),), i32), out_dtype=d.pick([bf, f32]))
  else:
    ops.ragged_dot_mxfp8_mxfp4(q, qs, wp, ws, _t((d.near(g),), i32), fuse_gateup_activation=d.pick([None, "situ:4:25"]),
                               out_dtype=d.pick([bf, f32]))


def _router(d):
  t, e = d.dim(), d.pick([8, 16, 64, 128])
  k = d.pick([1, 2, 8, 16, e, e + 1])
  bias = _t((d.near(e),), f32) if d.pick([True, False]) else None
  if d.pick([True, False]):
    ops.router_topk_from_logits(_t((d.near(t), d.near(e)), d.pick([f32, f32, bf])), bias, k,
                                weight_dtype=d.pick([f32, bf]), return_scores=d.pick([False, True]),
                                act=d.pick(["sigmoid", "softmax"]))
  else:
    lat = d.pick([8, 16, 64])
    wide = _t((d.near(t), e + lat + d.pick([0, 4])), f32)
    ops.router_topk_project(wide[:, :d.near(e)], wide[:, e:e + d.near(lat)], bias, k, weight_dtype=d.pick([f32, bf]))


def _dispatch(d):
  t, k, lat, L = d.dim(), d.pick([1, 2, 4, 16]), d.pick([8, 16, 64]), d.pick([1, 4, 16])
  m_padded = d.pick([0, 8, 64, 128, 256])
  idx, w = _t((t, k), i32), _t((d.near(t), d.near(k)), d.pick([f32, bf]))
  x = _t((d.near(t), d.near(lat)), d.pick([bf, f32])) if d.pick([True, True, False]) else None
  if d.pick([True, False]):
    ops.dispatch_local(idx, w, x, d.pick([0, 3]), L, m_padded, path=d.pick(["auto", "sort", "small"]),
                       skip_padding_rows=d.pick([False, True]), gather_rows=d.pick([True, True, False]),
                       lat=d.pick([None, lat]))
  else:
    n = d.pick([16, 32, 64])
    kk = d.pick([64, 128])
    xs = _t((d.near(t), d.near(kk)), bf)
    ops.dispatch_ragged_dot_mxfp4_skinny(idx, w, xs, 0, L, m_padded,
                                         _t((d.near(L + 1), d.near(kk // 64), d.near(n), 32), u8),
                                         _t((d.near(L + 1), d.near(kk // 64), d.near(n), 2), u8),
                                         fuse_gateup_activation=d.pick([None, "situ:4:25"]))


def _combine(d):
  t, k, lat, m = d.dim(), d.pick([1, 2, 4]), d.pick([8, 16, 64]), d.pick([0, 1, 8, 64])
  dt = d.pick([bf, f32])
  mode = d.pick(["slot_sum", "scatter_add"])
  shard = _t((d.near(m), d.near(lat)), dt)
  slot = _t((d.near(t), d.near(k)), i32)
  w = _t((d.near(t), d.near(k)), f32) if mode == "slot_sum" else _t((d.near(m),), dt)
  which = d.pick([0, 1, 2])
  if which == 0:
    routed = _t((d.near(t), d.near(lat)), dt) if d.pick([False, True]) else None
    ops.combine_slots(shard, slot, w, d.near(t), d.near(k), mode=mode, routed_out=routed,
                      out_dtype=d.pick([None, dt]))
  elif which == 1:
    ops.combine_slots_rms_norm(shard, slot, w, d.near(t), d.near(k), _t((d.near(lat),), dt), 1e-6, mode=mode,
                               out_dtype=d.pick([None, dt]), return_routed=d.pick([False, True]))
  else:
    ops._combine_shard_contribution(_t((d.near(t), d.near(lat)), dt), shard, _t((d.near(m),), i32),
                                    _t((d.near(m),), dt))


def _elementwise(d):
  r, n = d.dim(), d.pick([8, 16, 64, 256])
  dt = d.pick([bf, f32])
  which = d.pick(["norm", "situ", "add", "cast", "dense"])
  if which == "norm":
    ops._rms_norm(_t((d.near(r), d.near(n)), dt), _t((d.near(n),), d.pick([dt, dt, f32])), 1e-6)
  elif which == "situ":
    ops._situ_and_mul(_t((d.near(r), d.near(n)), dt), _t((d.near(r), d.near(n)), dt), 4.0, 25.0)
  elif which == "add":
    ops.add(_t((d.near(r), d.near(n)), dt), _t((d.near(r), d.near(n)), d.pick([dt, bf, f32])))
  elif which == "cast":
    wide = _t((d.near(r), n + d.pick([0, 8])), dt)
    ops.cast_rows(wide[:, :d.near(n)], d.pick([bf, f32]))
  else:
    k = d.pick([64, 128, 256])
    layout = d.pick(["kn", "nk"])
    w = _t((d.near(k), d.near(n)) if layout == "kn" else (d.near(n), d.near(k)), bf)
    ops.dense(_t((d.near(r), d.near(k)), bf), w, out_dtype=d.pick([None, f32]), w_layout=layout,
              backend=d.pick([None, "hip", "blaslt", "dense", "skinny"]))


CASES = {f.__name__[1:]: f for f in (_ragged_dot, _gateup, _fp8, _mxfp4, _mx_prep, _scaled, _router, _dispatch,
                                      _combine, _elementwise)}
# more examples where many tensors must agree for a call to go through
EXAMPLES = {"mxfp4": 800, "dispatch": 500, "fp8": 500}


@pytest.mark.parametrize("case", sorted(CASES))
def test_operators_on_arbitrary_shapes(monkeypatch, case):
  """Each operator either raises before a library call it cannot size, or
  every call it makes passes buffers that hold what its sizes say."""
  log = ExtentLog(monkeypatch)
  stats = {"called": 0, "refused": 0}

  @settings(max_examples=EXAMPLES.get(case, 250), deadline=None, derandomize=True, database=None,
            suppress_health_check=[HealthCheck.too_slow, HealthCheck.function_scoped_fixture])
  @given(st.data())
  def run(data):
    log.clear()
    try:
      CASES[case](_Draw(data))
    except (ValueError, NotImplementedError, TypeError, RuntimeError, IndexError):
      stats["refused"] += 1
    stats["called"] += bool(log.calls)
    check_extents(log.calls)

  run()
  print(case, stats)
  assert stats["called"] >= 40, stats  # the fuzz reaches the library, not only the refusals
