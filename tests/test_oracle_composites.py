"""The oracle's composite functions pinned against independent brute force:
the [gate | up] prefuse layout (rd.py:610-641; plain concatenation on N, not
interleaved, rd.py:204-233), the fused gate/up + SiTU-GLU (rd.py:644-723,
gk.py:114-125: accumulators rounded to bf16 before the activation) and the
MXFP4 matmul's orientation (odq.py:1-36: y = x @ deq(W)^T for W (N, K/2))
against float64 dot products over the OCP E2M1 value table.  Each check fails
on a plausible slip: an interleaved prefuse, gate and up swapped, the
nibbles of a byte decoded high-first, a transposed weight orientation; the
round-before-activation flag is shown to change the bf16 result."""
import numpy as np
import pytest

from oracle import lmoe_oracle as O

E2M1 = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])


def _situ64(g, u, b, bl):
  g, u = np.asarray(g, np.float64), np.asarray(u, np.float64)
  return b * np.tanh(g / b) / (1 + np.exp(-g)) * bl * np.tanh(u / bl)


def test_prefuse_is_gate_then_up_on_n():
  gate = np.arange(2 * 3 * 4, dtype=np.float32).reshape(2, 3, 4)
  up = -1 - np.arange(2 * 3 * 4, dtype=np.float32).reshape(2, 3, 4)
  fused = O.prefuse_gateup_weights(gate, up)
  assert fused.shape == (2, 3, 8)
  assert np.array_equal(fused[..., :4], gate) and np.array_equal(fused[..., 4:], up)
  # not interleaved: column 1 is gate column 1, not up column 0
  assert fused[0, 0, 1] == gate[0, 0, 1] != up[0, 0, 0]


def _brute_gateup(lhs, wg, wu, gs, b, bl, round_first=True):
  out = np.zeros((lhs.shape[0], wg.shape[-1]))
  start = 0
  for gi, n in enumerate(gs):
    for r in range(start, start + n):
      g = np.array([sum(float(lhs[r, k]) * float(wg[gi, k, j]) for k in range(lhs.shape[1]))
                    for j in range(wg.shape[-1])])
      u = np.array([sum(float(lhs[r, k]) * float(wu[gi, k, j]) for k in range(lhs.shape[1]))
                    for j in range(wu.shape[-1])])
      if round_first:
        g, u = O.bf16_round(g), O.bf16_round(u)
      out[r] = _situ64(g, u, b, bl)
    start += n
  return out


def test_fused_gateup_situ_against_brute_force():
  rng = np.random.default_rng(0)
  gs = np.array([3, 0, 4, 2], np.int32)
  m, k, inter, b, bl = 11, 16, 6, 4.0, 25.0
  lhs = O.bf16_round(rng.standard_normal((m, k)))
  wg = O.bf16_round(rng.standard_normal((4, k, inter)))
  wu = O.bf16_round(rng.standard_normal((4, k, inter)) * 0.3)
  got = O.ragged_dot_gateup_situ(lhs, O.prefuse_gateup_weights(wg, wu), gs, b, bl, "bf16").astype(np.float64)
  want = _brute_gateup(lhs, wg, wu, gs, b, bl)
  valid = int(gs.sum())
  # the oracle's f32 SiTU and final bf16 rounding: within 2 bf16 ulp of the f64 value
  scale = np.maximum(np.abs(want[:valid]), 1e-3)
  assert np.max(np.abs(got[:valid] - want[:valid]) / scale) <= 2 * 2.0 ** -8
  assert not got[valid:].any()  # rows past sum(group_sizes)
  # planted slips fail the same bound
  swapped = _brute_gateup(lhs, wu, wg, gs, b, bl)
  assert np.max(np.abs(got[:valid] - swapped[:valid]) / scale) > 0.1
  # the round-before-activation flag is honoured (for bf16; rounding to f32 is the identity)
  unrounded = O.ragged_dot_gateup_situ(lhs, O.prefuse_gateup_weights(wg, wu), gs, b, bl, "bf16",
                                       round_before_act=False)
  assert not np.array_equal(unrounded, got.astype(np.float32))


def _dequant_brute(packed, scale, k):
  n = packed.shape[0]
  w = np.zeros((n, k))
  for r in range(n):
    for j in range(k):
      byte = int(packed[r, j // 2])
      nib = byte & 15 if j % 2 == 0 else byte >> 4  # low nibble = element 2i
      v = E2M1[nib & 7] * (-1 if nib & 8 else 1)
      w[r, j] = v * 2.0 ** (int(scale[r, j // 32]) - 127)
  return w


def test_mxfp4_matmul_orientation_and_values():
  rng = np.random.default_rng(1)
  m, n, k = 5, 12, 64  # N != K: a transposed orientation cannot even multiply
  packed = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
  scale = rng.integers(120, 131, (n, k // 32), dtype=np.uint8)
  x = O.bf16_round(rng.standard_normal((m, k)))
  got = O.mxfp4_matmul(x, packed, scale, "f32").astype(np.float64)
  w = _dequant_brute(packed, scale, k)
  want = x.astype(np.float64) @ w.T
  assert got.shape == (m, n)
  assert np.max(np.abs(got - want)) <= 1e-5 * np.max(np.abs(x) @ np.abs(w).T)
  # the nibble order matters: high-nibble-first decoding gives another product
  swapped = ((packed >> 4) | (packed << 4)).astype(np.uint8)
  assert np.max(np.abs(O.mxfp4_matmul(x, swapped, scale, "f32") - want)) > 1e-2


@pytest.mark.parametrize("v,t,want", [(0, 128, 0), (1, 128, 128), (128, 128, 128), (129, 128, 256), (5, 4, 8)])
def test_round_up_to_tile(v, t, want):
  assert O.round_up_to_tile(v, t) == want


def test_grouped_mxfp4_with_situ_against_brute_force():
  """The grouped MXFP4 oracle with the SiTU epilogue (the config-5 gate/up:
  N = [gate | up] of each checkpoint expert, rd.py:610-723 on MXFP4 weights):
  per-row float64 dots over the E2M1 table, rounded to bf16 before a float64
  SiTU, within 2 bf16 ulp; the padding rows past sum(group_sizes) are zero."""
  rng = np.random.default_rng(2)
  gs = np.array([2, 0, 3, 1], np.int32)
  m, inter, k, b, bl = 8, 6, 64, 4.0, 25.0
  packed = rng.integers(0, 256, (4, 2 * inter, k // 2), dtype=np.uint8)
  scale = rng.integers(118, 124, (4, 2 * inter, k // 32), dtype=np.uint8)
  x = O.bf16_round(rng.standard_normal((m, k)))
  got = O.ragged_dot_mxfp4(x, packed, scale, gs, "bf16", situ=(b, bl)).astype(np.float64)
  want = np.zeros((m, inter))
  start = 0
  for g, n in enumerate(gs):
    w = _dequant_brute(packed[g], scale[g], k)
    for r in range(start, start + n):
      acc = x[r].astype(np.float64) @ w.T
      want[r] = _situ64(O.bf16_round(acc[:inter]), O.bf16_round(acc[inter:]), b, bl)
    start += int(n)
  valid = int(gs.sum())
  scale_ = np.maximum(np.abs(want[:valid]), 1e-3)
  assert got.shape == (m, inter)
  assert np.max(np.abs(got[:valid] - want[:valid]) / scale_) <= 2 * 2.0 ** -8
  assert not got[valid:].any()
