"""Pins of the oracle's MXFP6 (OCP MX FP6 E2M3 + E8M0) activation format,
used by the scaled-MFMA path at the FP4/FP6 rate.  No torch dtype exists for
FP6, so each function is checked against the OCP value table, a brute-force
nearest-value search and closed forms."""
import itertools

import numpy as np

from oracle import lmoe_oracle as O

# OCP MX v1.0 FP6 E2M3 magnitudes in code order: subnormals 0..7/8, then
# 1..15/8 (step 1/8), 2..3.75 (step 1/4), 4..7.5 (step 1/2)
TABLE = np.array([j / 8 for j in range(16)] + [2 + j / 4 for j in range(8)] + [4 + j / 2 for j in range(8)])


def test_e2m3_decode_matches_the_value_table():
  codes = np.arange(64)
  v = O.fp6_e2m3_to_f32(codes).astype(np.float64)
  assert np.array_equal(v[:32], TABLE)
  assert np.array_equal(v[32:], -TABLE)
  assert np.all(np.diff(v[:32]) > 0)  # monotone in the code
  assert v.max() == O.E2M3_MAX


def _nearest_even(a):
  """Brute force: the nearest table value, ties to the even code."""
  d = np.abs(TABLE[None, :] - a[:, None])
  best = d.min(axis=1, keepdims=True)
  cand = d == best
  codes = np.argmax(cand & (np.arange(32)[None, :] % 2 == 0), axis=1)
  only = cand.sum(axis=1) == 1
  codes = np.where(only, np.argmax(cand, axis=1), codes)
  return codes


def test_e2m3_encode_brute_force_with_every_midpoint():
  mids = (TABLE[1:] + TABLE[:-1]) / 2
  a = np.concatenate([np.linspace(0, 7.5, 30001), TABLE, mids, np.nextafter(mids, 0), np.nextafter(mids, 9)])
  got = O.f32_to_fp6_e2m3(a).astype(np.int64)
  assert np.array_equal(got, _nearest_even(a))
  neg = O.f32_to_fp6_e2m3(-a).astype(np.int64)
  assert np.array_equal(neg, _nearest_even(a) | 0x20)
  sat = O.f32_to_fp6_e2m3(np.array([7.6, 8.0, 1e30, np.inf, -np.inf, np.nan]))
  assert list(sat) == [31, 31, 31, 31, 63, 0]


def test_quantize_mxfp6_exponent_and_round_trip():
  rng = np.random.default_rng(3)
  x = rng.standard_normal((16, 256)) * 10.0 ** rng.integers(-20, 20, (16, 1))
  x[0, :32] = 0.0
  codes, scales = O.quantize_mxfp6(x)
  amax = np.abs(x.reshape(16, 8, 32)).max(axis=-1)
  ex = scales.astype(np.int64) - 127
  nz = amax > 0
  ratio = amax[nz] / np.ldexp(1.0, ex[nz])
  assert np.all((ratio >= 4) & (ratio < 8))  # floor(log2 amax) - 2
  assert scales[0, 0] == 0
  # values already on the scaled grid round-trip exactly
  grid_codes = rng.integers(0, 64, (4, 64))
  grid_scale = rng.integers(100, 150, (4, 2)).astype(np.uint8)
  vals = O.dequantize_mxfp6(grid_codes, grid_scale)
  # force a block maximum of magnitude >= 4 so the chosen exponent is the given one
  vals[:, 0] = 7.5 * np.ldexp(1.0, grid_scale[:, 0].astype(np.int64) - 127)
  vals[:, 32] = 4.0 * np.ldexp(1.0, grid_scale[:, 1].astype(np.int64) - 127)
  c2, s2 = O.quantize_mxfp6(vals)
  assert np.array_equal(s2, grid_scale)
  assert np.array_equal(O.dequantize_mxfp6(c2, s2), vals)


def test_quantize_mxfp6_planted_emax_mistake_fails():
  """The MX choice floor(log2 amax) - 2 keeps every element within its grid
  bound; floor(log2 amax) - 3 saturates the block maximum far past it."""
  rng = np.random.default_rng(4)
  x = rng.standard_normal((8, 128))
  codes, scales = O.quantize_mxfp6(x)
  err = np.abs(O.dequantize_mxfp6(codes, scales) - x)
  # half the largest grid spacing (1/2 of the scale), or, for the elements in
  # (7.5, 8) x scale that saturate, at most a whole spacing
  step = np.repeat(np.ldexp(1.0, scales.astype(np.int64) - 127 - 1), 32, axis=-1)
  sat = np.abs(x) > 7.5 * 2 * step
  assert np.all(err[~sat] <= step[~sat] / 2)
  assert np.all(err[sat] <= step[sat])
  blocks = x.reshape(8, 4, 32)
  amax = np.abs(blocks).max(axis=-1)
  bad_ex = (np.floor(np.log2(amax)) - 3).astype(np.int64)
  bad = O.fp6_e2m3_to_f32(O.f32_to_fp6_e2m3(blocks * np.ldexp(1.0, -bad_ex)[..., None])) * np.ldexp(1.0, bad_ex)[..., None]
  assert np.any(np.abs(bad - blocks).reshape(8, 128) > step)


def test_fp6_packing_bit_placement_and_round_trip():
  for j in range(32):
    c = np.zeros((1, 32), np.uint8)
    c[0, j] = 0x3F
    p = O.pack_fp6(c)[0]
    bits = np.unpackbits(p, bitorder="little")
    assert np.array_equal(np.nonzero(bits)[0], np.arange(6 * j, 6 * j + 6))
  rng = np.random.default_rng(5)
  codes = rng.integers(0, 64, (3, 128)).astype(np.uint8)
  assert np.array_equal(O.unpack_fp6(O.pack_fp6(codes), 128), codes)


def test_ragged_dot_mxfp6_mxfp4_brute_force():
  rng = np.random.default_rng(6)
  m, k, n, g = 7, 64, 5, 2
  codes = rng.integers(0, 64, (m, k)).astype(np.uint8)
  sc = rng.integers(120, 134, (m, k // 32)).astype(np.uint8)
  wp = rng.integers(0, 256, (g, n, k // 2), dtype=np.uint8)
  ws = rng.integers(120, 134, (g, n, k // 32), dtype=np.uint8)
  gs = np.array([4, 2], np.int32)
  got = O.ragged_dot_mxfp6_mxfp4(codes, sc, wp, ws, gs, "f32")
  want = np.zeros((m, n))
  r0 = 0
  for gi, cnt in enumerate(gs):
    wd = O.dequantize_mxfp4(wp[gi], ws[gi])
    for r, c in itertools.product(range(r0, r0 + cnt), range(n)):
      want[r, c] = sum(float(O.fp6_e2m3_to_f32(codes[r, kk])) * 2.0 ** (int(sc[r, kk // 32]) - 127) * float(wd[c, kk])
                       for kk in range(k))
    r0 += cnt
  assert np.array_equal(got, want.astype(np.float32))
