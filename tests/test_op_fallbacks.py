"""The operators' host-side routes around what the kernels take, checked for
values on the CPU with the emulating library stand-in (the oracle's
definitions behind the C-ABI): a bf16 ragged_dot whose K or N is off the
bf16 kernels' 8-element grid runs the f32 kernel on the same values and
rounds once (bit for bit the oracle's bf16 ragged_dot); an f32 or off-grid
fused gate/up runs its two halves and the SiTU-GLU (the oracle's fused
gate/up, with and without rounding before the activation); empty problems
(M, N or K = 0, e.g. a layer without shared experts) return their zero or
empty output without a library call."""
import numpy as np
import pytest
import torch

import _emulated_lib
from _util import to_np
from lmoe import ops
from oracle import lmoe_oracle as O

bf = torch.bfloat16


def _t(a, dt):
  t = torch.from_numpy(np.ascontiguousarray(a, np.float32))
  return t.to(bf) if dt == "bf16" else t


@pytest.mark.parametrize("k,n,layout", [(12, 60, "gkn"), (64, 60, "gnk"), (12, 64, "gkn"), (8, 2, "gnk")])
def test_off_grid_bf16_ragged_dot_is_the_oracles(monkeypatch, k, n, layout):
  lib = _emulated_lib.install(monkeypatch)
  rng = np.random.default_rng(k * n)
  gs = np.array([5, 0, 9, 3], np.int32)
  lhs = O.bf16_round(rng.standard_normal((20, k)))
  rhs = O.bf16_round(rng.standard_normal((4, k, n)))
  want = O.ragged_dot(lhs, rhs, gs, "bf16")
  w = rhs if layout == "gkn" else np.ascontiguousarray(rhs.transpose(0, 2, 1))
  got = ops.ragged_dot(_t(lhs, "bf16"), _t(w, "bf16"), torch.from_numpy(gs), rhs_layout=layout)
  assert got.dtype == bf and np.array_equal(to_np(got), want)
  assert lib.names() == ["lmoe_ragged_dot"]
  # f32 output: the f32 kernel's result itself
  got32 = ops.ragged_dot(_t(lhs, "bf16"), _t(w, "bf16"), torch.from_numpy(gs), rhs_layout=layout,
                         preferred_element_type=torch.float32)
  assert np.array_equal(to_np(got32), O.ragged_dot(lhs, rhs, gs, "f32"))


@pytest.mark.parametrize("shape", [(0, 16, 8), (6, 0, 8), (6, 16, 0)])
def test_empty_ragged_dot(monkeypatch, shape):
  lib = _emulated_lib.install(monkeypatch)
  m, k, n = shape
  out = ops.ragged_dot(torch.ones(m, k, dtype=bf), torch.ones(2, k, n, dtype=bf),
                       torch.tensor([m, 0], dtype=torch.int32))
  assert out.shape == (m, n) and not out.float().abs().sum() and not lib.names()


@pytest.mark.parametrize("backend", [None, "hip", "blaslt", "dense", "skinny"])
def test_empty_dense(monkeypatch, backend):
  lib = _emulated_lib.install(monkeypatch)
  for m, k, n in ((0, 128, 4096), (4, 0, 4096), (4, 128, 0)):
    out = ops.dense(torch.ones(m, k, dtype=bf), torch.ones(n, k, dtype=bf), w_layout="nk", backend=backend)
    assert out.shape == (m, n) and not out.float().abs().sum()
  assert not lib.names()


def test_shared_expert_mlp_of_width_zero(monkeypatch):
  """A layer without shared experts: the shared MLP's matrices are (H, 0) /
  (0, H), its output zeros, the residual add unchanged (the reference's
  zero-width matmuls)."""
  _emulated_lib.install(monkeypatch)
  x = _t(np.random.default_rng(0).standard_normal((5, 64)), "bf16")
  z = ops._situ_glu_mlp(x, torch.zeros(64, 0, dtype=bf), torch.zeros(64, 0, dtype=bf),
                        torch.zeros(0, 64, dtype=bf), 4.0, 25.0)
  assert z.shape == (5, 64) and not z.float().abs().sum()
  assert torch.equal(ops.add(x, z), x)


@pytest.mark.parametrize("dt,inter,round_first", [("f32", 16, True), ("f32", 12, True), ("bf16", 12, True),
                                                  ("bf16", 12, False), ("bf16", 20, True)])
@pytest.mark.parametrize("layout", ["gkn", "gnk"])
def test_fused_gateup_routes(monkeypatch, dt, inter, round_first, layout):
  """The f32 and off-grid fused gate/up against the oracle's fused gate/up:
  [gate | up] halves taken from the right side of the prefused weight."""
  lib = _emulated_lib.install(monkeypatch)
  rng = np.random.default_rng(inter)
  gs = np.array([4, 0, 7], np.int32)
  lhs = O.cast(rng.standard_normal((13, 24)), dt)
  wg, wu = O.cast(rng.standard_normal((3, 24, inter)), dt), O.cast(rng.standard_normal((3, 24, inter)) * 0.3, dt)
  fused = O.prefuse_gateup_weights(wg, wu)
  want = O.ragged_dot_gateup_situ(lhs, fused, gs, 4.0, 25.0, dt, round_before_act=round_first)
  w = fused if layout == "gkn" else np.ascontiguousarray(fused.transpose(0, 2, 1))
  got = ops.ragged_dot_gateup_situ(_t(lhs, dt), _t(w, dt), torch.from_numpy(gs), 4.0, 25.0, rhs_layout=layout,
                                   round_before_act=round_first)
  assert got.dtype == (bf if dt == "bf16" else torch.float32) and got.shape == (13, inter)
  # the halves are separate f32 products here, one product over [gate | up] in
  # the oracle: equal up to f32 summation order, i.e. within one output ulp
  tol = 2.0 ** -8 if dt == "bf16" else 1e-6
  np.testing.assert_allclose(to_np(got), want, rtol=tol, atol=tol * np.abs(want).max())
  assert lib.names() == ["lmoe_ragged_dot", "lmoe_ragged_dot", "lmoe_situ_and_mul"]
  # a swapped split (up first) is far off
  swapped = O.ragged_dot_gateup_situ(lhs, O.prefuse_gateup_weights(wu, wg), gs, 4.0, 25.0, dt)
  assert np.abs(to_np(got) - swapped).max() > 100 * tol * np.abs(want).max()
