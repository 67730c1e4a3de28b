"""Pins the oracle's MXFP8 (OCP MX E4M3 + E8M0, block 32) quantiser and the
MXFP8 x MXFP4 grouped GEMM used to check the native scaled-MFMA path.

The reference has no such path, so these checks anchor the oracle on a library
routine (torch.float8_e4m3fn casts), on the OCP MX closed form and on brute
force; a planted mistake in the exponent rule is rejected.
"""
import numpy as np
import pytest
import torch

from oracle import lmoe_oracle as O


def _torch_codes(x):
  return torch.from_numpy(np.clip(np.asarray(x, np.float32), -448, 448)).to(torch.float8_e4m3fn).view(
      torch.uint8).numpy()


def test_e4m3_decode_all_codes_vs_torch():
  codes = np.arange(256, dtype=np.uint8)
  mine = O.fp8_e4m3_to_f32(codes)
  ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
  nan = np.isnan(ref)
  assert np.array_equal(np.isnan(mine), nan) and nan.sum() == 2  # 0x7F, 0xFF
  assert np.array_equal(mine[~nan].view(np.uint32), ref[~nan].view(np.uint32))  # incl. -0.0
  assert mine[0x7E] == 448.0 and mine[0x01] == 2.0 ** -9


def test_e4m3_encode_rne_and_saturation_vs_torch():
  rng = np.random.default_rng(0)
  grid = O.fp8_e4m3_to_f32(np.arange(256, dtype=np.uint8))
  grid = np.sort(grid[~np.isnan(grid)])
  ties = (grid[:-1] + grid[1:]) / 2  # exact midpoints: ties to even
  x = np.concatenate([rng.standard_normal(100000) * 30, rng.standard_normal(50000) * 1e-2,
                      rng.standard_normal(20000) * 1e-3, grid, ties,
                      np.array([448.0, 449.0, 464.0, 480.0, 1e6, -1e6, 0.0, -0.0])]).astype(np.float32)
  assert np.array_equal(O.f32_to_fp8_e4m3(x), _torch_codes(x))
  assert O.f32_to_fp8_e4m3(np.array([np.inf, -np.inf, np.nan])).tolist() == [0x7E, 0xFE, 0x7F]


def _closed_form_check(quantize):
  rng = np.random.default_rng(1)
  x = (rng.standard_normal((37, 256)) * np.exp(rng.uniform(-12, 12, (37, 1)))).astype(np.float32)
  x[3, 32:64] = 0.0  # an all-zero block
  codes, scales = quantize(x)
  blocks = x.reshape(37, 8, 32).astype(np.float64)
  amax = np.abs(blocks).max(-1)
  expect = np.where(amax > 0, np.floor(np.log2(np.where(amax > 0, amax, 1))) - 8 + 127, 0)
  assert np.array_equal(scales.astype(np.int64), expect.astype(np.int64))
  deq = O.dequantize_mxfp8(codes, scales).reshape(37, 8, 32)
  # every element within half an E4M3 quantum of its scaled value, except the
  # block maxima above 448 * 2^e, which saturate to exactly 448 * 2^e
  scale = np.ldexp(1.0, scales.astype(np.int64) - 127)[..., None]
  rel = np.abs(deq - blocks) / scale
  quantum = np.ldexp(1.0, (np.maximum(np.floor(np.log2(np.maximum(np.abs(blocks) / scale, 2.0 ** -6))), -6) - 3)
                     .astype(np.int64))
  sat = np.abs(blocks) / scale > 448
  assert np.all((rel <= quantum / 2 + 1e-12) | sat)
  assert np.all(np.abs(deq[sat]) == 448 * np.broadcast_to(scale, deq.shape)[sat])
  assert np.all(codes.reshape(37, 8, 32)[3, 1] == 0)


def test_quantize_mxfp8_closed_form():
  _closed_form_check(O.quantize_mxfp8)


def test_quantize_mxfp8_grid_values_round_trip():
  rng = np.random.default_rng(2)
  codes = rng.integers(0, 256, (16, 128)).astype(np.uint8)
  codes[(codes & 0x7F) == 0x7F] = 0x7E  # no NaN
  codes[:, 1::32] = 0x79  # exp 15, mant 1 -> 1.125 * 2^8 = 288: block max in [256, 512), scale byte 127
  scales = np.full((16, 4), 127, np.uint8)
  x = O.dequantize_mxfp8(codes, scales)
  c2, s2 = O.quantize_mxfp8(x)
  assert np.array_equal(s2, scales)
  assert np.array_equal(O.dequantize_mxfp8(c2, s2), x)


def test_planted_exponent_mistake_is_caught():
  def wrong(x):  # emax off by one: scale 2x too large, elements lose a bit
    c, s = O.quantize_mxfp8(np.asarray(x, np.float64) / 2)
    return c, (s.astype(np.int64) + 1).astype(np.uint8)
  with pytest.raises(AssertionError):
    _closed_form_check(wrong)


def test_ragged_dot_mxfp8_mxfp4_brute_force():
  rng = np.random.default_rng(3)
  m, k, n, g = 7, 64, 5, 3
  gs = np.array([2, 0, 4], np.int32)  # one tail row
  a = rng.standard_normal((m, k)).astype(np.float32)
  codes, scales = O.quantize_mxfp8(a)
  packed = rng.integers(0, 256, (g, n, k // 2), dtype=np.uint8)
  wsc = rng.integers(120, 130, (g, n, k // 32), dtype=np.uint8)
  got = O.ragged_dot_mxfp8_mxfp4(codes, scales, packed, wsc, gs, "f32")
  ad = O.dequantize_mxfp8(codes, scales)
  ref = np.zeros((m, n))
  row = 0
  for gi, cnt in enumerate(gs):
    w = O.dequantize_mxfp4(packed[gi], wsc[gi]).astype(np.float64)
    for r in range(row, row + cnt):
      for c in range(n):
        ref[r, c] = sum(ad[r, kk] * w[c, kk] for kk in range(k))
    row += cnt
  assert np.allclose(got, ref.astype(np.float32), rtol=1e-6, atol=1e-6)
  assert np.all(got[6] == 0)


def test_mxfp8_path_equals_bf16_path_on_the_e4m3_grid():
  """Activations that are exactly representable in both E4M3 (with a block scale)
  and bf16 give the same GEMM through both oracles."""
  rng = np.random.default_rng(4)
  m, k, n, g = 33, 128, 24, 2
  codes = rng.integers(0x30, 0x48, (m, k)).astype(np.uint8) | (rng.integers(0, 2, (m, k)) << 7).astype(np.uint8)
  codes[:, ::32] = 0x78  # 256: block max in [256, 512)
  scales = rng.integers(118, 126, (m, k // 32)).astype(np.uint8)
  a = O.dequantize_mxfp8(codes, scales).astype(np.float32)
  assert np.array_equal(O.bf16_round(a), a)
  c2, s2 = O.quantize_mxfp8(a)
  assert np.array_equal(c2, codes) and np.array_equal(s2, scales)
  packed = rng.integers(0, 256, (g, n, k // 2), dtype=np.uint8)
  wsc = rng.integers(122, 128, (g, n, k // 32), dtype=np.uint8)
  gs = np.array([20, 13], np.int32)
  x = O.ragged_dot_mxfp8_mxfp4(codes, scales, packed, wsc, gs, "f32")
  y = O.ragged_dot_mxfp4(a, packed, wsc, gs, "f32")
  assert np.max(np.abs(x - y)) <= 1e-5 * np.max(np.abs(y))


@pytest.mark.parametrize("bs", [None, 32])
def test_fp8_blockscaled_dequant_matches_torch(bs):
  """(rhs_q.astype(f32) * scale).astype(bf16) (rd.py:2815, rd.py:2934-2935)
  through torch's own float8_e4m3fn -> f32 -> bf16 casts: all 256 codes in
  every column, per-column (bs = K) and 32-row block scales, including
  subnormal products and negative / zero scales."""
  rng = np.random.default_rng(8)
  g, k, n = 2, 256, 64
  codes = ((np.arange(k)[:, None] + 7 * np.arange(n)[None, :]) % 256).astype(np.uint8)
  codes = np.broadcast_to(codes, (g, k, n)).copy()
  nb = 1 if bs is None else k // bs
  scale = (rng.standard_normal((g, nb, 1, n)) * 10.0 ** rng.integers(-40, 30, (g, nb, 1, n))).astype(np.float32)
  scale[0, 0, 0, :4] = [0.0, -1.0, 1e-38, 2.0 ** -140]
  ours = O.dequantize_fp8_blockscaled(codes, scale)
  tq = torch.from_numpy(codes).view(torch.float8_e4m3fn).float()
  ts = torch.from_numpy(scale).repeat_interleave(k // nb, dim=1).reshape(g, k, n)
  theirs = (tq * ts).to(torch.bfloat16).float().numpy()
  nan = np.isnan(theirs)
  assert np.array_equal(np.isnan(ours), nan)
  assert np.array_equal(ours[~nan].view(np.uint32), theirs[~nan].view(np.uint32))


def test_fp8_scaled_ragged_dot_is_dequant_then_matmul():
  """The fp8 op equals ragged_dot on the dequantised bf16 weights (the
  reference's own comparison), checked against a per-row float64 brute force."""
  rng = np.random.default_rng(9)
  g, k, n = 3, 64, 24
  codes = rng.integers(0, 256, (g, k, n), dtype=np.uint8)
  codes[(codes & 0x7F) == 0x7F] = 0  # no NaN codes
  scale = (rng.uniform(0.5, 2.0, (g, 2, 1, n)) * 0.01).astype(np.float32)
  gs = np.array([5, 0, 7], np.int32)
  lhs = O.bf16_round(rng.standard_normal((14, k)))
  out = O.ragged_dot_fp8_scaled(lhs, codes, scale, gs, "f32")
  w = O.dequantize_fp8_blockscaled(codes, scale).astype(np.float64)
  rows = np.repeat(np.arange(g), gs)
  for r, grp in enumerate(rows):
    assert np.allclose(out[r], lhs[r].astype(np.float64) @ w[grp], rtol=1e-5, atol=1e-6)
  assert not out[len(rows):].any()
