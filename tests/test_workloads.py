"""Host-side workload generation: the OCP MX quantiser and the Zipf group sizes."""
import numpy as np
import pytest
import torch

from lmoe import workloads as W
from oracle import lmoe_oracle as O


def test_quantize_round_trips_representable_values():
  rng = np.random.default_rng(0)
  codes = rng.integers(0, 16, (4, 64))
  codes[:, ::32] = 7  # every block holds a 6.0 so the block amax fixes the exponent
  exps = rng.integers(-10, 10, (4, 2))
  vals = O.fp4_e2m1_to_f32(codes) * np.repeat(np.ldexp(1.0, exps), 32, axis=1).astype(np.float32)
  packed, scale = W.quantize_mxfp4(torch.from_numpy(vals))
  back = O.dequantize_mxfp4(packed.numpy(), scale.numpy())
  assert np.array_equal(back, vals)


def test_quantize_error_bound_and_ties():
  rng = np.random.default_rng(1)
  x = (rng.standard_normal((64, 256)) * 0.02).astype(np.float32)
  packed, scale = W.quantize_mxfp4(torch.from_numpy(x))
  back = O.dequantize_mxfp4(packed.numpy(), scale.numpy())
  amax = np.repeat(np.abs(x).reshape(64, 8, 32).max(-1), 32, axis=1)
  assert np.all(np.abs(back - x) <= amax / 2 + 1e-12)
  # ties to even: with scale 2^0 (block amax 4), 0.25 -> 0, 0.75 -> 1, 1.25 -> 1, 2.5 -> 2, 5 -> 4
  blk = np.zeros((1, 32), np.float32)
  blk[0, :6] = [4.0, 0.25, 0.75, 1.25, 2.5, 5.0]
  p, s = W.quantize_mxfp4(torch.from_numpy(blk))
  assert s.item() == 127
  assert O.dequantize_mxfp4(p.numpy(), s.numpy())[0, :6].tolist() == [4.0, 0.0, 1.0, 1.0, 2.0, 4.0]


def test_zipf_group_sizes():
  gs = W.zipf_group_sizes(8192, 32, seed=2)
  assert gs.sum() == 8192 and (gs == 0).sum() >= 3 and gs.dtype == np.int32
  assert gs.max() > 4 * 8192 / 32  # skewed


def test_harness_distributions_are_the_reference_vectors():
  """benchmark_harness.py:116-150, written out for G = 4: mild skew doubles
  group 0's weight, heavy skew gives it weight G, empty_groups zeroes the
  second half, single_dominant puts everything in group 0."""
  assert W.harness_distribution("uniform", 4) is None
  assert W.harness_distribution("mild_skew", 4) == [2 / 5, 1 / 5, 1 / 5, 1 / 5]
  assert W.harness_distribution("heavy_skew", 4) == [4 / 7, 1 / 7, 1 / 7, 1 / 7]
  assert W.harness_distribution("empty_groups", 4) == [0.5, 0.5, 0.0, 0.0]
  assert W.harness_distribution("empty_groups", 1) == [1.0]
  assert W.harness_distribution("single_dominant", 4) == [1.0, 0.0, 0.0, 0.0]
  with pytest.raises(ValueError):
    W.harness_distribution("zipf", 4)


@pytest.mark.parametrize("shape", list(W.HARNESS_SHAPES))
@pytest.mark.parametrize("dist", W.HARNESS_DISTRIBUTIONS)
def test_harness_group_sizes(shape, dist):
  m, _, _, g = W.HARNESS_SHAPES[shape]
  gs = W.harness_group_sizes(m, g, dist, seed=5)
  assert gs.dtype == np.int32 and gs.shape == (g,) and gs.sum() == m and gs.min() >= 0
  assert np.array_equal(gs, W.harness_group_sizes(m, g, dist, seed=5))  # seeded
  if dist == "uniform":
    assert gs.max() - gs.min() <= 1
  if dist == "empty_groups":
    assert np.all(gs[g // 2:] == 0) and np.all(gs[: g // 2] > 0)
  if dist == "single_dominant":
    assert gs[0] == m
  if dist in ("mild_skew", "heavy_skew"):
    # group 0's share within 5 binomial sigmas of its probability
    p0 = W.harness_distribution(dist, g)[0]
    assert abs(gs[0] - m * p0) <= 5 * np.sqrt(m * p0 * (1 - p0))


def test_global_picks_uniform_without_replacement():
  """Every token's picks are distinct, and over many tokens each expert is
  picked T*k/E times within a chi-square bound (uniform draw)."""
  rng = np.random.default_rng(3)
  t, e, k = 20000, 96, 8
  picks = W._draw_global_picks(rng, t, e, k)
  assert picks.shape == (t, k) and picks.min() >= 0 and picks.max() < e
  assert all(len(set(row)) == k for row in picks[:2000])
  assert np.all(np.sort(picks, 1)[:, 1:] != np.sort(picks, 1)[:, :-1])
  counts = np.bincount(picks.reshape(-1), minlength=e)
  expect = t * k / e
  chi2 = float(((counts - expect) ** 2 / expect).sum())
  assert chi2 < e + 6 * np.sqrt(2 * e), chi2  # ~6 sigma above the mean of chi2(e-1)
  # each position is uniform too (the order within a token is random)
  first = np.bincount(picks[:, 0], minlength=e)
  assert float(((first - t / e) ** 2 / (t / e)).sum()) < e + 6 * np.sqrt(2 * e)


@pytest.mark.parametrize("t,e,k,L,cf", [(4096, 896, 16, 112, 2.0), (300, 64, 6, 16, 1.5), (1, 896, 16, 112, 2.0),
                                        (512, 64, 8, 32, 1.0)])
def test_generate_local_shard_workload_invariants(t, e, k, L, cf):
  """ref.py:474-598: fixed m_padded = round_up(ceil(T*k*L/E*cf), 128) (the
  oracle's m_padded formula), per-expert counts as drawn (truncated from the
  tail on overflow), one padding bucket, zero padding rows, valid mask on the
  kept rows."""
  lat = 64
  st, gs, valid, counts = W.generate_local_shard_workload(t, e, k, L, lat, capacity_factor=cf, seed=t, device="cpu")
  m_padded = O.compute_m_padded(t, k, e, L, cf)
  assert st.shape == (m_padded, lat) and st.dtype == torch.bfloat16
  gs, counts, valid = gs.numpy(), counts.numpy(), valid.numpy()
  assert gs.shape == (L + 1,) and gs.dtype == np.int32 and gs.sum() == m_padded
  assert np.array_equal(gs[:L], counts)
  keep = int(counts.sum())
  assert valid.sum() == keep and valid[:keep].all() and not valid[keep:].any()
  assert not st[keep:].float().abs().sum() and (st[:keep].float().abs().sum(1) > 0).all()
  # the draw itself: the same seeded picks, kept below L, sorted, truncated
  picks = W._draw_global_picks(np.random.default_rng(t), t, e, k).reshape(-1)
  raw = np.sort(picks[picks < L])
  assert np.array_equal(counts, np.bincount(raw[:m_padded], minlength=L))
  if raw.size > m_padded:
    # overflow drops the tail: the highest expert ids lose picks first
    full = np.bincount(raw, minlength=L)
    lost = np.nonzero(full != counts)[0]
    assert lost.size and np.array_equal(full[:lost[0]], counts[:lost[0]])
    assert not counts[lost[0] + 1:].any()
