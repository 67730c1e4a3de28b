"""The fused GEMM epilogue's SiTU-GLU formula (``situ_epi`` in
csrc/gemm_tile.h) on the CPU: a float32 model with the device's operation
order, clamps and beta == 4 identity -- exactly rounded exp2 and reciprocal in
place of the hardware's (a few ulp apart, covered by the GPU tests) -- checked
against the SiTU of ref.py:296-310 in float64 over the whole range of gate and
up values, including the far-negative gate range g in [-100, -36] where the
beta == 4 sigmoid saturates at 2^-52.  The error bound is the one the kernel
source states: a few f32 ulp relative, plus beta*beta_lin*2^-23 absolute
(cancellation of a - 1 near 0), plus beta*beta_lin*2^-52 for the saturated
sigmoid.  Variants with a plausible slip (a narrower clamp, sigmoid written as
a/(1+a)) fail the same bound."""
import numpy as np
import pytest

from oracle import lmoe_oracle as O

F32 = np.float32
L2E = F32(1.44269504088896341)


def situ_epi_model(g, u, beta, beta_lin, clamp=26.0, beta4_identity="a2"):
  """float32 restatement of gemm_tile.h situ_epi (fmed3 clamp, exp2, rcp)."""
  g, u = np.asarray(g, F32), np.asarray(u, F32)
  kg = F32(2.0) * L2E / F32(beta)
  ku = F32(2.0) * L2E / F32(beta_lin)
  bbl = F32(beta) * F32(beta_lin)
  c = F32(clamp)
  with np.errstate(over="ignore", under="ignore", invalid="ignore", divide="ignore"):
    a = np.exp2(np.clip(g * kg, -c, c)).astype(F32)
    b = np.exp2(np.clip(u * ku, -c, c)).astype(F32)
    one = F32(1.0)
    if F32(beta) == F32(4.0):
      a2 = a * a if beta4_identity == "a2" else a
      r = bbl * ((a - one) * a2 * (b - one)) * (one / ((a + one) * (one + a2) * (b + one)))
    else:
      e = np.exp2(g * -L2E).astype(F32)
      q = (a - one) * (b - one) * (one / ((a + one) * (b + one)))
      r = bbl * q * (one / (one + e))
  return np.where(np.isnan(g) | np.isnan(u), F32(np.nan), r).astype(F32)


def situ_f64(g, u, beta, beta_lin):
  g, u = np.asarray(g, np.float64), np.asarray(u, np.float64)
  with np.errstate(over="ignore"):
    sig = 1.0 / (1.0 + np.exp(-g))
  return beta * np.tanh(g / beta) * sig * beta_lin * np.tanh(u / beta_lin)


def _grid():
  g = np.concatenate([np.linspace(-100, 100, 2001), np.linspace(-100, -36, 641), np.linspace(-1e-3, 1e-3, 201),
                      [-88.7, -87.3, -36.0, -35.9, 0.0, 36.0, 88.7]]).astype(F32)
  u = np.concatenate([np.linspace(-200, 200, 401), np.linspace(-1e-3, 1e-3, 41), [0.0]]).astype(F32)
  return np.meshgrid(g, u, indexing="ij")


def _excess(r, beta, beta_lin, g, u, rel=2.0 ** -20):
  """How far the model lies outside the stated bound (<= 0: inside)."""
  ref = situ_f64(g, u, beta, beta_lin)
  bbl = beta * beta_lin
  bound = rel * np.abs(ref) + bbl * 2.0 ** -23 + bbl * 2.0 ** -52
  return float(np.max(np.abs(r.astype(np.float64) - ref) - bound))


@pytest.mark.parametrize("beta,beta_lin", [(4.0, 25.0), (4.0, 1.0), (2.0, 25.0), (8.0, 10.0), (1.0, 1.0)])
def test_epilogue_formula_within_its_stated_bound(beta, beta_lin):
  g, u = _grid()
  r = situ_epi_model(g, u, beta, beta_lin)
  assert np.all(np.isfinite(r))
  assert _excess(r, beta, beta_lin, g, u) <= 0.0
  # the same rows through the oracle's f32 SiTU (rounded to f32, not bf16)
  ref32 = O.situ_and_mul(g, u, beta, beta_lin, "f32")
  scale = beta * beta_lin
  assert np.max(np.abs(r - ref32) - 2.0 ** -19 * np.abs(ref32)) <= scale * 2.0 ** -22


def test_far_negative_gate_saturates_at_2_to_minus_52_with_beta_4():
  """g in [-100, -36] with beta == 4: sigmoid(g) = a^2 / (1 + a^2) with a =
  e^(g/2) clamped at 2^-26 (reached at g = -26 * 2 / log2(e) = -36.04) stays
  at 2^-52 below that, so the result is at most beta*beta_lin*max(2^-52,
  sigmoid(g)) in magnitude, and exactly the floor
  -beta*beta_lin*2^-52*tanh(u/beta_lin) once a is clamped.  Relative slack
  2^-17: the f32 exponent g*kg (about -26) carries an absolute rounding of
  26 * 2^-24, i.e. about 2^-19 relative in e^(g/2)."""
  beta, beta_lin = 4.0, 25.0
  g = np.linspace(-100, -36, 6401).astype(F32)[:, None]
  u = np.array([-200, -25, -1, 1, 25, 200], F32)[None, :]
  r = situ_epi_model(g, u, beta, beta_lin).astype(np.float64)
  sig = 1.0 / (1.0 + np.exp(-g.astype(np.float64)))
  assert np.all(np.abs(r) <= beta * beta_lin * np.maximum(2.0 ** -52, sig) * (1 + 2.0 ** -17))
  g_sat = -26.0 * beta / (2.0 * float(L2E))
  assert -36.05 < g_sat < -36.03
  below = g[:, 0] < g_sat
  floor = -beta * beta_lin * 2.0 ** -52 * np.tanh(u.astype(np.float64) / beta_lin)
  assert np.allclose(r[below], np.broadcast_to(floor, r[below].shape), rtol=2.0 ** -17, atol=0)


def test_nan_in_either_input_gives_nan():
  r = situ_epi_model(np.array([np.nan, 1.0], F32), np.array([1.0, np.nan], F32), 4.0, 25.0)
  assert np.all(np.isnan(r))


@pytest.mark.parametrize("variant", [{"clamp": 13.0}, {"beta4_identity": "a"}])
def test_a_slip_in_the_formula_fails_the_bound(variant):
  g, u = _grid()
  r = situ_epi_model(g, u, 4.0, 25.0, **variant)
  assert _excess(r, 4.0, 25.0, g, u) > 0.0
