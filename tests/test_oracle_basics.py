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


def test_gate_exp64_against_libm():
  """The router's binary64 exp (Cody-Waite reduction + degree-13 Taylor) is
  within 1 ulp of the C library's exp over the whole clamped range, exact at
  0 and 1 ulp-close at integers; outside the range it saturates to inf / 0."""
  t = np.concatenate([np.linspace(-708.0, 709.0, 400001), np.linspace(-1.0, 1.0, 200001),
                      np.arange(-708.0, 710.0)])
  e = O.gate_exp64(t)
  ulp = np.abs(e - np.exp(t)) / np.spacing(np.exp(t))
  assert ulp.max() <= 1.0, ulp.max()
  assert O.gate_exp64(0.0) == 1.0
  assert abs(O.gate_exp64(1.0) - math.e) <= 2 * np.spacing(math.e)
  edge = O.gate_exp64(np.array([709.5, 1e300, np.inf, -708.5, -1e300, -np.inf, np.nan]))
  assert np.array_equal(edge[:6], [np.inf] * 3 + [0.0] * 3) and np.isnan(edge[6])


def test_gate_exp64_planted_mistakes_fail():
  """Dropping the low part of ln2 or the two highest Taylor terms breaks the
  1-ulp bound."""
  t = np.linspace(-700.0, 700.0, 100001)
  good = np.abs(O.gate_exp64(t) - np.exp(t)) / np.spacing(np.exp(t))
  assert good.max() <= 1.0
  saved = (O.GATE_LN2_LO, O.GATE_INV_FACT)
  try:
    O.GATE_LN2_LO = 0.0
    assert (np.abs(O.gate_exp64(t) - np.exp(t)) / np.spacing(np.exp(t))).max() > 100
    O.GATE_LN2_LO = saved[0]
    O.GATE_INV_FACT = saved[1][:12] + (0.0, 0.0)
    assert (np.abs(O.gate_exp64(t) - np.exp(t)) / np.spacing(np.exp(t))).max() > 4
  finally:
    O.GATE_LN2_LO, O.GATE_INV_FACT = saved


def test_gate_sigmoid_is_correctly_rounded():
  """f32 sigmoid within half an f32 ulp of the extended-precision value (so
  correctly rounded) on a wide sample, including subnormal results, +-0,
  +-inf and saturation."""
  rng = np.random.default_rng(4)
  x = np.concatenate([rng.standard_normal(400000) * 6, rng.uniform(-110, 40, 100000),
                      [0.0, -0.0, 88.7, -87.3, -100.0, -103.97, -200.0, 1e30, -1e30, np.inf, -np.inf]])
  x = x.astype(np.float32)
  s = O.gate_sigmoid(x)
  with np.errstate(over="ignore"):
    ld = 1 / (1 + np.exp(-x.astype(np.longdouble)))
  half = np.spacing(np.abs(s)).astype(np.longdouble) / 2
  tiny = np.longdouble(2.0) ** -149  # subnormal spacing
  assert np.all(np.abs(s.astype(np.longdouble) - ld) <= np.maximum(half, tiny / 2) * (1 + 1e-6))
  assert O.gate_sigmoid(np.float32(0)) == 0.5 and O.gate_sigmoid(np.float32(np.inf)) == 1.0
  assert O.gate_sigmoid(np.float32(-np.inf)) == 0.0 and O.gate_sigmoid(np.float32(-100)) > 0


def test_gate_softmax_closed_form():
  """Within one f32 ulp of the extended-precision softmax of the f32
  differences x - max (the gate subtracts in f32), rows sum to 1, and E not a
  multiple of 64 (padding partials) works."""
  rng = np.random.default_rng(5)
  for e_n in (8, 64, 100, 896, 4096):
    x = (rng.standard_normal((32, e_n)) * 4).astype(np.float32)
    p = O.gate_softmax(x)
    d = (x - x.max(-1, keepdims=True)).astype(np.float32).astype(np.longdouble)
    ref = np.exp(d)
    ref /= ref.sum(-1, keepdims=True)
    assert np.all(np.abs(p - ref) <= np.spacing(p).astype(np.longdouble)), e_n
    assert np.allclose(p.astype(np.float64).sum(-1), 1.0, atol=1e-6)


def test_router_renorm_sums_in_topk_order():
  """The renormalisation divides by the f32 sum of the chosen scores taken in
  top-k order (j = 0, 1, ...): checked on values where that order and a
  pairwise sum round differently."""
  logits = np.zeros((1, 4), np.float32)
  scores = np.array([0.5, 2.0 ** -25, 2.0 ** -25, 0.25], np.float32)
  logits[0] = -np.log(1 / scores.astype(np.float64) - 1)
  r = O.router_from_logits(logits, np.array([0, 0, 0, 0], np.float32), 4, True, 1.0)
  s = O.gate_sigmoid(logits)[0][r.topk_idx[0]]
  seq = np.float32(0)
  for v in s:
    seq = np.float32(seq + v)
  assert np.array_equal(r.topk_weight[0], (s / (seq + np.float32(1e-20))).astype(np.float32))


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


def test_bits_to_f32_every_bf16_pattern():
  """All 65536 bf16 bit patterns: decoded as torch's bfloat16 view decodes
  them, and (NaNs aside) encoded back to the same bits by ``bf16_bits``;
  ``cast`` is ``bf16_round`` for bf16 and the identity on float32."""
  u = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
  got = O.bits_to_f32(u)
  theirs = torch.from_numpy(u.view(np.int16)).view(torch.bfloat16).float().numpy()
  assert np.array_equal(got.view(np.uint32), theirs.view(np.uint32))
  finite = ~np.isnan(got)
  assert np.array_equal(O.bf16_bits(got[finite]), u[finite])
  assert np.isnan(O.bits_to_f32(O.bf16_bits(got[~finite]))).all()
  x = np.random.default_rng(7).standard_normal(1000).astype(np.float32)
  assert np.array_equal(O.cast(x, "bf16"), torch.from_numpy(x).bfloat16().float().numpy())
  assert np.array_equal(O.cast(x, "f32"), x)


def test_promote_matches_torch():
  t = {"bf16": torch.bfloat16, "f32": torch.float32}
  for a in t:
    for b in t:
      assert t[O.promote(a, b)] == torch.promote_types(t[a], t[b]), (a, b)


def test_matmul_rounds_once_from_f32_accumulation():
  rng = np.random.default_rng(8)
  a = O.bf16_round(rng.standard_normal((33, 200)))
  b = O.bf16_round(rng.standard_normal((200, 17)))
  exact = a.astype(np.float64) @ b.astype(np.float64)
  acc_err = 200 * 2.0 ** -24 * (np.abs(a).astype(np.float64) @ np.abs(b))  # f32 accumulation bound
  f32 = O.matmul(a, b, "f32")
  assert f32.dtype == np.float32 and np.all(np.abs(f32 - exact) <= acc_err)
  bf = O.matmul(a, b, "bf16")
  half_ulp = 2.0 ** (np.floor(np.log2(np.abs(exact))) - 8)
  assert np.array_equal(bf, O.bf16_round(bf)) and np.all(np.abs(bf - exact) <= half_ulp + 2 * acc_err)


def test_e8m0_and_e2m1_decoders_every_code():
  """OCP MX v1.0: an E8M0 byte s is 2^(s-127) (byte 0 the float32 denormal
  2^-127; 255 overflows float32 to inf as the reference's 2^(s-127) does),
  an E2M1 nibble is given by ``_e2m1_spec``."""
  s = np.arange(256)
  got = O.e8m0_to_f32(s.astype(np.uint8))
  with np.errstate(over="ignore"):
    want = np.array([np.float32(math.ldexp(1.0, int(v) - 127)) for v in s[:255]] + [np.float32(np.inf)])
  assert got.dtype == np.float32 and np.array_equal(got, want)
  codes = np.arange(16, dtype=np.uint8)
  got = O.fp4_e2m1_to_f32(codes)
  want = np.array([_e2m1_spec(int(c)) for c in codes], np.float32)
  assert np.array_equal(got, want) and np.array_equal(np.signbit(got), codes >= 8)


def test_every_public_oracle_function_is_pinned():
  """``PINNING`` names every public function of the oracle, and nothing else."""
  import inspect
  public = {n for n, f in vars(O).items()
            if inspect.isfunction(f) and f.__module__ == O.__name__ and not n.startswith("_")}
  named = [n.strip() for key in O.PINNING for n in key.split(" / ")]
  assert len(named) == len(set(named))
  assert set(named) == public, (sorted(public - set(named)), sorted(set(named) - public))
