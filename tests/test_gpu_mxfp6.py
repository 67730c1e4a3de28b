"""GPU parity: the scaled-MFMA path at the FP4/FP6 rate (MXFP6 E2M3 activations
x MXFP4 weights on v_mfma_scale_f32_32x32x64_f8f6f4) against the oracle's OCP
MX definition.

* quantisation: packed codes and E8M0 scales bit-exact (zero blocks, NaN,
  +-inf, saturation, subnormal inputs, values far below a block's range);
* GEMM with f32 output against the exact (float64) dot of the dequantised
  operands: |d| <= 2^-14 * sum_k |a_k w_k| elementwise, the bar of the MXFP8
  path (the instruction does not accumulate its block dot in full fp32); a
  wrong lane mapping, packing or scale misses it by orders of magnitude;
* rows past the groups and of the zero group are zero.
The deviation of this path from the bf16 reference path (activations not
quantised) is printed for the record; it is a property of MXFP6.
"""
import numpy as np
import pytest
import torch

from _util import banner, max_rel, to_dev, to_np
from oracle import lmoe_oracle as O

pytestmark = pytest.mark.gpu


def _scales_checkpoint(scale_t, m):
  """(K/128, M4, 4) -> (M, K/32)."""
  s = to_np(scale_t)
  return np.ascontiguousarray(s.transpose(1, 0, 2).reshape(s.shape[1], -1)[:m])


@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_quantize_mxfp6_bit_exact(gpu_device, dt):
  from lmoe import ops
  rng = np.random.default_rng(21)
  m, k = 101, 384
  x = (rng.standard_normal((m, k)) * np.exp(rng.uniform(-30, 30, (m, 1)))).astype(np.float32)
  x[0, :32] = 0.0                               # zero block
  x[1, 5] = np.nan                              # NaN element
  x[1, 6] = -np.nan
  x[2, 7], x[2, 8] = np.inf, -np.inf            # infinities: excluded from amax, saturate
  x[3, :32] = np.float32(2.0 ** -130)           # subnormal block
  x[4, 40:64] = 1e-30                           # elements far below the block's range
  x[5, :32] = np.float32(1.0)                   # amax 1: scale 2^-2, so x * 4 is rounded
  x[5, 1:4] = [0.078125, 0.53125, 1.0625]       # ties after scaling: 2.5/8, 8.5/4, 8.5/2 -> even codes
  x = O.cast(x, dt)
  q, sc = ops.quantize_mxfp6(to_dev(x, dt))
  codes, scales = O.quantize_mxfp6(x)
  got = to_np(q)
  assert got.shape == (m, k * 3 // 4)
  assert np.array_equal(got, O.pack_fp6(codes))
  assert np.array_equal(_scales_checkpoint(sc, m), scales)
  assert np.all(to_np(sc)[:, m:, :] == 0)  # pad rows of the k-step-major layout


def _abs_dot(a64, packed, wsc, gs):
  a = np.abs(a64)
  out = np.zeros((a.shape[0], packed.shape[1]))
  start = 0
  for g, n in enumerate(gs):
    if n:
      out[start:start + n] = a[start:start + n] @ np.abs(O.dequantize_mxfp4(packed[g], wsc[g]).astype(np.float64)).T
    start += int(n)
  return out


MX6_CASES = [
    # m, k, n, g, tail rows, zero_group
    (300, 256, 128, 5, 17, -1),
    (64, 128, 8, 1, 0, -1),        # narrowest N: one partial n-tile
    (333, 7168, 256, 1, 0, -1),    # config-4 depth
    (1024, 1024, 384, 9, 5, 8),    # trailing zero group
    (130, 2048, 1024, 4, 3, 3),
    (1, 7168, 2048, 1, 0, -1),     # one row
    (4096, 7168, 2048, 1, 0, -1),  # BASELINE config 4 at the size its throughput is quoted at
]


@pytest.mark.parametrize("m,k,n,g,tail,zg", MX6_CASES)
def test_ragged_dot_mxfp6_mxfp4_f32(gpu_device, m, k, n, g, tail, zg):
  from lmoe import ops
  banner(f"mxfp6 x mxfp4 m={m} k={k} n={n} g={g} zero_group={zg}")
  rng = np.random.default_rng(m + k + n + g + 1)
  gs = rng.multinomial(m - tail, np.ones(g) / g).astype(np.int32)
  if g > 2:
    gs[1] = 0
  a = O.bf16_round(rng.standard_normal((m, k)))
  if zg >= 0:
    start = int(gs[:zg].sum())
    a[start:start + gs[zg]] = 0.0
  packed = rng.integers(0, 256, (g, n, k // 2), dtype=np.uint8)
  wsc = rng.integers(119, 130, (g, n, k // 32), dtype=np.uint8)
  codes, scales = O.quantize_mxfp6(a)
  ref = O.ragged_dot_mxfp6_mxfp4(codes, scales, packed, wsc, gs, "f32")
  q, qs = ops.quantize_mxfp6(to_dev(a, "bf16"))
  tpk, tsc = ops.mxfp4_tile_weights(to_dev(packed), to_dev(wsc))
  out = ops.ragged_dot_mxfp6_mxfp4(q, qs, tpk, tsc, to_dev(gs), zero_group=zg, out_dtype=torch.float32)
  o = to_np(out)
  assert o.shape == ref.shape
  absum = _abs_dot(O.dequantize_mxfp6(codes, scales), packed, wsc, gs)
  bad = np.abs(o - ref) > 2.0 ** -14 * absum
  rel = np.abs(o - ref) / np.maximum(absum, 1e-300)
  print(f"  worst |d| / sum|a w| = 2^{np.log2(max(rel.max(), 1e-300)):.1f}; violations {int(bad.sum())}")
  assert not bad.any()
  assert np.all(o[int(gs.sum()):] == 0)
  if zg >= 0:
    start = int(gs[:zg].sum())
    assert np.all(o[start:start + gs[zg]] == 0)
  via = ops.ragged_dot_mxfp4(to_dev(a, "bf16"), tpk, tsc, to_dev(gs), mode="scaled_mfma_fp6", zero_group=zg,
                             weight_layout="tiled")
  assert torch.equal(via, out.to(torch.bfloat16))
  bf16_path = O.ragged_dot_mxfp4(a, packed, wsc, gs, "f32")
  print(f"  deviation of MXFP6 activations from the bf16 path: {max_rel(o, bf16_path):.3e}")


def test_mxfp6_mode_limits(gpu_device):
  from lmoe import ops
  a = torch.zeros((64, 128), dtype=torch.bfloat16, device="cuda")
  pk = torch.zeros((1, 2, 64, 32), dtype=torch.uint8, device="cuda")
  sc = torch.zeros((1, 2, 64, 2), dtype=torch.uint8, device="cuda")
  gs = torch.tensor([64], dtype=torch.int32, device="cuda")
  with pytest.raises(NotImplementedError):
    ops.ragged_dot_mxfp4(a, pk, sc, gs, mode="scaled_mfma_fp6", weight_layout="tiled",
                         fuse_gateup_activation="situ:4.0:25.0")
  with pytest.raises(NotImplementedError):
    ops.quantize_mxfp6(torch.zeros((4, 96), dtype=torch.bfloat16, device="cuda"))
