"""The operators, for values, on the CPU: each runs against the emulating
stand-in library (the oracle's definition of every entry point behind the
real library's host checks) and its result is compared with the oracle's
own function on the same inputs -- so what is checked is the operator's
side of the contract: which entry point with which sizes, layouts, scales,
casts and views.  Covered: ``dense`` on every backend and weight layout,
the op class ``HipRaggedDot`` for each weight kind (bf16, fused gate/up,
block-scaled fp8, MXFP4 checkpoint / tiled / skinny, MXFP4 with MXFP8
activations), the MXFP4 split-K and gathered-rows forms, the reference-named
dispatch and routing entry points, the scatter-add combine, MXFP4
dequantisation and the router on row-strided logits.  Bit for bit wherever
the oracle and the emulated entry point compute the same arithmetic."""
import numpy as np
import pytest
import torch

import _emulated_lib
from _util import to_np
from lmoe import ops
from lmoe.config import LatentMoEConfig
from oracle import lmoe_oracle as O

bf = torch.bfloat16


def _t(a, dt="bf16"):
  t = torch.from_numpy(np.ascontiguousarray(a)).clone()
  return t.to(bf) if dt == "bf16" else t


@pytest.fixture
def lib(monkeypatch):
  return _emulated_lib.install(monkeypatch)


RNG = np.random.default_rng(5)
GS = np.array([5, 0, 9, 2], np.int32)
M, K, N, G = 16, 128, 64, 4


def _mx(n=N, k=K, g=G):
  packed = RNG.integers(0, 256, (g, n, k // 2), dtype=np.uint8)
  scale = RNG.integers(118, 130, (g, n, k // 32), dtype=np.uint8)
  return packed, scale


@pytest.mark.parametrize("backend,layout", [(None, "kn"), (None, "nk"), ("hip", "kn"), ("hip", "nk"),
                                            ("blaslt", "nk"), ("dense", "nk"), ("skinny", "nk")])
@pytest.mark.parametrize("out", [None, torch.float32])
def test_dense(lib, backend, layout, out):
  x = O.bf16_round(RNG.standard_normal((4, K)))
  w = O.bf16_round(RNG.standard_normal((K, N)) * 0.1)
  got = ops.dense(_t(x), _t(w if layout == "kn" else w.T), out_dtype=out, w_layout=layout, backend=backend)
  assert np.array_equal(to_np(got), O.matmul(x, w, "f32" if out == torch.float32 else "bf16"))


def test_op_class_weight_kinds(lib):
  op = ops.HipRaggedDot()
  lhs = O.bf16_round(RNG.standard_normal((M, K)))
  gs = torch.from_numpy(GS)
  # bf16 weights, and the fused gate/up on [gate | up]
  w = O.bf16_round(RNG.standard_normal((G, K, N)) * 0.1)
  assert np.array_equal(to_np(op(_t(lhs), _t(w), group_sizes=gs)), O.ragged_dot(lhs, w, GS, "bf16"))
  assert np.array_equal(to_np(op(_t(lhs), _t(w), group_sizes=gs, fuse_gateup_activation="situ:4:25")),
                        O.ragged_dot_gateup_situ(lhs, w, GS, 4.0, 25.0, "bf16"))
  # block-scaled fp8 weights, one scale per 32 rows of K
  q = RNG.integers(0, 256, (G, K, N), dtype=np.uint8)
  q[(q & 0x7F) == 0x7F] = 0  # no NaN codes
  sc = RNG.uniform(0.5, 2.0, (G, K // 32, 1, N)).astype(np.float32)
  got = op(_t(lhs), torch.from_numpy(q).view(torch.float8_e4m3fn), group_sizes=gs, rhs_scale=_t(sc, "f32"))
  assert np.array_equal(to_np(got), O.ragged_dot_fp8_scaled(lhs, q, sc, GS, "bf16"))
  # MXFP4 weights: checkpoint layout, tiled with the fused gate/up, and MXFP8 activations
  packed, scale = _mx()
  want = O.ragged_dot_mxfp4(lhs, packed, scale, GS, "bf16")
  assert np.array_equal(to_np(op(_t(lhs), _t(packed, "u8"), group_sizes=gs, rhs_scale=_t(scale, "u8"))), want)
  tp, ts = ops.mxfp4_tile_weights(_t(packed, "u8"), _t(scale, "u8"))
  assert np.array_equal(to_np(op(_t(lhs), tp, group_sizes=gs, rhs_scale=ts, fuse_gateup_activation="situ:4:25")),
                        O.ragged_dot_mxfp4(lhs, packed, scale, GS, "bf16", situ=(4.0, 25.0)))
  assert np.array_equal(to_np(ops.HipRaggedDot(mxfp4_mode="skinny")(_t(lhs), tp, group_sizes=gs, rhs_scale=ts)),
                        want)
  codes, scales = O.quantize_mxfp8(lhs)
  got = op(_t(lhs), _t(packed, "u8"), group_sizes=gs, rhs_scale=_t(scale, "u8"), maybe_quantize_lhs=True)
  assert np.array_equal(to_np(got), O.ragged_dot_mxfp8_mxfp4(codes, scales, packed, scale, GS, "bf16"))


def test_mxfp4_split_k_and_gathered_rows(lib):
  packed, scale = _mx(g=1, k=512)
  tp, ts = ops.mxfp4_tile_weights(_t(packed, "u8"), _t(scale, "u8"))
  lhs = O.bf16_round(RNG.standard_normal((M, 512)))
  one = torch.tensor([M], dtype=torch.int32)
  got = ops.ragged_dot_mxfp4(_t(lhs), tp, ts, one, weight_layout="tiled", k_split=3)
  assert lib.names()[-1] == "lmoe_ragged_dot_mxfp4_splitk"
  assert np.array_equal(to_np(got), O.ragged_dot_mxfp4(lhs, packed, scale, [M], "bf16"))
  tokens = O.bf16_round(RNG.standard_normal((7, 512)))
  idx = RNG.integers(0, 7, M).astype(np.int32)
  got = ops.ragged_dot_mxfp4(_t(tokens), tp, ts, one, weight_layout="tiled", lhs_row_index=torch.from_numpy(idx))
  assert lib.names()[-1] == "lmoe_ragged_dot_mxfp4_rows"
  assert np.array_equal(to_np(got), O.ragged_dot_mxfp4(tokens[idx], packed, scale, [M], "bf16"))


def test_mxfp4_dequant(lib):
  packed, scale = _mx()
  for dt, name in ((torch.float32, "f32"), (bf, "bf16")):
    got = ops.dequantize_mxfp4(_t(packed, "u8"), _t(scale, "u8"), out_dtype=dt)
    assert np.array_equal(to_np(got), O.cast(O.dequantize_mxfp4(packed, scale), name))


@pytest.mark.parametrize("jittable", [False, True])
def test_reference_named_dispatch_and_routing(lib, jittable):
  cfg = LatentMoEConfig(hidden_size=64, latent_size=32, intermediate_size=32, num_experts=32, top_k=4,
                        num_shared_experts=0)
  t, start, L = 40, 8, 8
  hidden = O.bf16_round(RNG.standard_normal((t, 64)))
  router = O.bf16_round(RNG.standard_normal((64, 32)) * 0.1)
  bias = np.zeros(32, np.float32)
  x = O.bf16_round(RNG.standard_normal((t, 32)))
  r, _ = O.router_gate(hidden, router, bias, cfg, weight_dtype="bf16")
  want = O.filter_and_pad_to_shard_jittable(r.topk_idx, r.topk_weight, x, 4, 32, start, L)
  fn = ops.route_and_filter_to_local_shard_jittable if jittable else ops.route_and_filter_to_local_shard
  got = fn(_t(hidden), _t(x), _t(router), _t(bias, "f32"), cfg, start, L)
  for name, a, b in zip(want._fields, got, want):
    assert np.array_equal(to_np(a), b), name
  fn = ops.filter_and_pad_to_shard_jittable if jittable else ops.filter_and_pad_to_shard
  got = fn(torch.from_numpy(r.topk_idx), _t(r.topk_weight), _t(x), cfg, start, L)
  for name, a, b in zip(want._fields, got, want):
    assert np.array_equal(to_np(a), b), name


def test_scatter_add_combine(lib):
  t, m, lat = 9, 24, 16
  routed = O.bf16_round(RNG.standard_normal((t, lat)))
  shard = O.bf16_round(RNG.standard_normal((m, lat)))
  idx = RNG.integers(-1, t, m).astype(np.int32)
  w = O.bf16_round(RNG.uniform(size=m))
  got = ops._combine_shard_contribution(_t(routed), _t(shard), torch.from_numpy(idx), _t(w))
  assert np.array_equal(to_np(got), O.combine_shard_contribution(routed, shard, idx, w, "bf16", "bf16", "bf16"))


@pytest.mark.parametrize("act", ["sigmoid", "softmax"])
def test_router_on_a_row_slice(lib, act):
  wide = RNG.standard_normal((12, 40 + 24)).astype(np.float32)
  bias = RNG.standard_normal(40).astype(np.float32) * 0.01
  idx, w, scores = ops.router_topk_from_logits(_t(wide, "f32")[:, :40], _t(bias, "f32"), 6, act=act,
                                               return_scores=True)
  r = O.router_from_logits(wide[:, :40], bias, 6, True, 1.0, act)
  assert np.array_equal(to_np(idx), r.topk_idx) and np.array_equal(to_np(w), r.topk_weight)
  assert np.array_equal(to_np(scores), r.scores)


@pytest.mark.parametrize("gather_rows", [True, False])
def test_dispatch_with_no_capacity(lib, gather_rows):
  """m_padded = 0 with tokens routed (a capacity factor of 0): every slot is
  dropped -- zero group sizes and counts, every slot_pos -1 -- as the oracle
  gives it, with no library call."""
  t, k, L = 6, 2, 4
  idx = np.stack([RNG.permutation(8)[:k] for _ in range(t)]).astype(np.int32)
  w = RNG.uniform(size=(t, k)).astype(np.float32)
  x = O.bf16_round(RNG.standard_normal((t, 16)))
  want, slot_pos = O.filter_and_pad_to_shard_jittable(idx, w, x, k, 8, 0, L, m_padded=0, return_slot_pos=True)
  got = ops.dispatch_local(torch.from_numpy(idx), _t(w, "f32"), _t(x), 0, L, 0, gather_rows=gather_rows, lat=16)
  assert lib.names() == []
  for name, a, b in zip(want._fields, got, want):
    if a is None:
      assert name == "sorted_tokens" and not gather_rows
      continue
    assert tuple(a.shape) == b.shape and np.array_equal(to_np(a), b), name
  assert np.array_equal(to_np(got.slot_pos), slot_pos)
