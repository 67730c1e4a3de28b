"""Host-side workload generation: the OCP MX quantiser and the Zipf group sizes."""
import numpy as np
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
