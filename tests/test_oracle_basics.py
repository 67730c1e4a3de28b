"""Pins the oracle's elementwise pieces against independent formulations:
bf16 rounding vs torch's cast, top_k vs brute force, softmax/SiTU/RMSNorm
closed forms in float64, MXFP4 decode vs the OCP MX v1.0 bit formula, and
planted-mistake checks showing the golden comparison rejects plausible bugs."""
import math

import numpy as np
import pytest
import torch

import _golden
from oracle import lmoe_oracle as O


def test_bf16_round_matches_torch_cast():
  rng = np.random.default_rng(0)
  x = np.concatenate([
      rng.standard_normal(100000).astype(np.float32),
      (rng.standard_normal(10000) * 1e-38).astype(np.float32),  # denormals
      np.array([0.0, -0.0, np.inf, -np.inf, 3.4e38, -3.4e38, 1 + 2 ** -8, 1 + 3 * 2 ** -8], np.float32),
      rng.integers(0, 2 ** 32, 100000, dtype=np.uint64).astype(np.uint32).view(np.float32),
  ])
  x = x[~np.isnan(x)]
  ours = O.bf16_bits(x)
  theirs = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
  assert np.array_equal(ours, theirs)


def test_bf16_ties_to_even():
  assert O.bf16_round(np.float32(1 + 2 ** -8)) == 1.0  # tie -> even (down)
  assert O.bf16_round(np.float32(1 + 3 * 2 ** -8)) == np.float32(1 + 2 ** -6)  # tie -> even (up)


def test_top_k_ties_lower_index_first():
  v = np.array([[0.5, 0.9, 0.5, 0.9, 0.1]], np.float32)
  assert O.top_k(v, 3).tolist() == [[1, 3, 0]]
  rng = np.random.default_rng(1)
  v = rng.integers(0, 5, (200, 40)).astype(np.float32)
  got = O.top_k(v, 7)
  for row, g in zip(v, got):
    brute = sorted(range(40), key=lambda e: (-row[e], e))[:7]
    assert g.tolist() == brute


def test_softmax_and_sigmoid_closed_form():
  rng = np.random.default_rng(2)
  x = rng.standard_normal((16, 896)).astype(np.float32) * 3
  x64 = x.astype(np.float64)
  sm = np.exp(x64 - x64.max(-1, keepdims=True))
  sm /= sm.sum(-1, keepdims=True)
  assert np.max(np.abs(O.softmax(x) - sm) / sm) < 1e-5
  assert np.max(np.abs(O.sigmoid(x) - 1 / (1 + np.exp(-x64)))) < 1e-6


def test_situ_closed_form():
  g = np.linspace(-30, 30, 2001).astype(np.float32)
  u = np.linspace(40, -40, 2001).astype(np.float32)
  ref = 4 * np.tanh(g / 4.0) / (1 + np.exp(-g.astype(np.float64))) * (25 * np.tanh(u / 25.0))
  assert np.max(np.abs(O.situ_and_mul(g, u, 4.0, 25.0, "f32") - ref)) < 1e-4


def test_rms_norm_closed_form():
  rng = np.random.default_rng(3)
  x = rng.standard_normal((8, 128)).astype(np.float32)
  s = rng.standard_normal(128).astype(np.float32)
  x64 = x.astype(np.float64)
  ref = x64 / np.sqrt((x64 ** 2).mean(-1, keepdims=True) + 1e-5) * s
  assert np.max(np.abs(O.rms_norm(x, s, 1e-5, "f32") - ref)) < 1e-5


def _e2m1_spec(code):
  """OCP MX v1.0 E2M1: sign bit 3, exponent bits 2:1 (bias 1), mantissa bit 0;
  exponent 0 is subnormal (0.m * 2^0)."""
  e, m = (code >> 1) & 3, code & 1
  mag = 0.5 * m if e == 0 else math.ldexp(1.0 + 0.5 * m, e - 1)
  return -mag if code & 8 else mag


def test_mxfp4_dequant_exhaustive_vs_spec():
  bytes_ = np.arange(256, dtype=np.uint8)
  for s in (0, 1, 100, 119, 126, 127, 128, 129, 200, 254, 255):
    packed = bytes_.reshape(1, 256)
    scale = np.full((1, 512 // 32), s, np.uint8)
    out = O.dequantize_mxfp4(packed, scale)[0]
    for b in range(256):
      for half, code in ((0, b & 15), (1, b >> 4)):
        v = _e2m1_spec(code)
        with np.errstate(over="ignore", invalid="ignore"):
          expect = np.float32(np.float64(v) * math.ldexp(1.0, s - 127)) if s < 255 else (
              np.float32(v) * np.float32(np.inf))
        got = out[2 * b + half]
        if np.isnan(expect):
          assert np.isnan(got)
        else:
          assert got == expect and np.signbit(got) == np.signbit(expect), (s, b, half)


def test_mxfp4_dequant_literal_kat():
  # byte 0x2F: low nibble 0xF = -6, high nibble 0x2 = +1; byte 0x80: +0, -0
  packed = np.array([[0x2F, 0x80] + [0] * 14], np.uint8)
  out = O.dequantize_mxfp4(packed, np.array([[128]], np.uint8))[0]
  assert out[:4].tolist() == [-12.0, 2.0, 0.0, -0.0] and np.signbit(out[3])


def test_mxfp4_scale_group_is_32_along_k():
  packed = np.full((2, 32), 0x22, np.uint8)  # all ones
  scale = np.array([[127, 128], [129, 126]], np.uint8)
  out = O.dequantize_mxfp4(packed, scale)
  assert np.all(out[0, :32] == 1) and np.all(out[0, 32:] == 2)
  assert np.all(out[1, :32] == 4) and np.all(out[1, 32:] == 0.5)


def test_ragged_dot_brute_force():
  rng = np.random.default_rng(4)
  gs = np.array([3, 0, 5, 1, 0], np.int32)
  lhs = rng.standard_normal((10, 6)).astype(np.float32)  # 9 rows used, 1 trailing
  rhs = rng.standard_normal((5, 6, 4)).astype(np.float32)
  out = O.ragged_dot(lhs, rhs, gs, "f32")
  grp = np.repeat(np.arange(5), gs)
  for r in range(10):
    for c in range(4):
      expect = sum(float(lhs[r, k]) * float(rhs[grp[r], k, c]) for k in range(6)) if r < 9 else 0.0
      assert abs(out[r, c] - expect) < 1e-5


# ---------------------------------------------------------------------------
# Planted mistakes: each plausible bug in the oracle must fail the golden check.
# ---------------------------------------------------------------------------

def _golden_failures(bundle="golden_bundle_small"):
  config, dtype, hidden, w, golden = _golden.load(bundle)
  w = {k: O.cast(v, dtype) for k, v in w.items()}
  _, inter = O.latent_moe_forward(hidden, w, config, dtype)
  atol, rtol = _golden.TOLERANCES[dtype]
  bad = []

  def check(name, g, o, exact):
    if g.shape != o.shape or (exact and not np.array_equal(g, o)) or (
        not exact and not np.allclose(g, o, atol=atol, rtol=rtol)):
      bad.append(name)

  _golden.compare_stages(golden, inter, config, dtype, check)
  return bad


@pytest.mark.parametrize("mutation", ["no_renorm", "swap_gate_up", "situ_sign", "norm_eps", "bias_in_weight"])
def test_planted_mistake_is_caught(monkeypatch, mutation):
  assert _golden_failures() == []
  if mutation == "no_renorm":
    orig = O.router_from_logits
    monkeypatch.setattr(O, "router_from_logits",
                        lambda l, b, k, r, s, a="sigmoid", wd="f32": orig(l, b, k, False, s, a, wd))
  elif mutation == "swap_gate_up":
    orig = O.situ_and_mul
    monkeypatch.setattr(O, "situ_and_mul", lambda g, u, b, lb, d: orig(u, g, b, lb, d))
  elif mutation == "situ_sign":
    orig = O.sigmoid
    monkeypatch.setattr(O, "sigmoid", lambda x: orig(-np.asarray(x)))
  elif mutation == "norm_eps":
    orig = O.rms_norm
    monkeypatch.setattr(O, "rms_norm", lambda x, s, e, d: orig(x, s, 1.0, d))
  elif mutation == "bias_in_weight":
    orig = O.router_from_logits

    def with_bias(l, b, k, r, s, a="sigmoid", wd="f32"):
      out = orig(l, b, k, r, s, a, wd)
      w = np.take_along_axis(out.scores_for_choice, out.topk_idx.astype(np.int64), -1)
      w = w / (w.sum(-1, keepdims=True) + 1e-20)
      return out._replace(topk_weight=w.astype(np.float32))
    monkeypatch.setattr(O, "router_from_logits", with_bias)
  assert _golden_failures() != []
