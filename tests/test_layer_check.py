"""The layer checks' routing-agreement bound (tests/_layer_check.py
``check_flips``) on the CPU: routing that differs only where a measured logit
perturbation can reorder near-tied selection keys is accepted, at any count;
a token routed to an expert whose key lies further below than the
perturbation explains is rejected, even if it is the only one."""
import numpy as np
import pytest

from _layer_check import check_flips, gate_lipschitz
from oracle import lmoe_oracle as O

T, E, K = 256, 128, 8


def _logits_with_ties(rng, eps):
  """N(0, 1) logits where every token's k-th and (k+1)-th largest (and its
  first and second largest) logits are eps apart, so a perturbation of a few
  eps can swap them."""
  lg = rng.standard_normal((T, E)).astype(np.float32)
  order = np.argsort(-lg, axis=1)
  rows = np.arange(T)
  lg[rows, order[:, K]] = lg[rows, order[:, K - 1]] - np.float32(eps)
  lg[rows, order[:, 1]] = lg[rows, order[:, 0]] - np.float32(eps)
  return lg


@pytest.mark.parametrize("act", ["sigmoid", "softmax"])
def test_near_ties_flipped_by_the_logit_error_are_accepted(act):
  rng = np.random.default_rng(7)
  lg_own = _logits_with_ties(rng, 2e-6)
  bias = np.zeros(E, np.float32)
  own = O.router_from_logits(lg_own, bias, K, True, 1.0, act)
  # another summation order: every logit moved by up to 8e-6
  lg_dev = (lg_own + rng.uniform(-8e-6, 8e-6, lg_own.shape)).astype(np.float32)
  dev = O.router_from_logits(lg_dev, bias, K, True, 1.0, act)
  differ = check_flips(dev.topk_idx, own.topk_idx, lg_dev, lg_own, own.scores_for_choice, act)
  # the construction flips many tokens, both at the k-th place and inside the top-k
  assert differ > T // 10, differ


@pytest.mark.parametrize("act", ["sigmoid", "softmax"])
def test_a_flip_the_logit_error_cannot_explain_is_rejected(act):
  rng = np.random.default_rng(8)
  lg_own = rng.standard_normal((T, E)).astype(np.float32)
  bias = (rng.standard_normal(E) * 0.1).astype(np.float32)
  own = O.router_from_logits(lg_own, bias, K, True, 1.0, act)
  lg_dev = (lg_own + rng.uniform(-1e-6, 1e-6, lg_own.shape)).astype(np.float32)
  dev = O.router_from_logits(lg_dev, bias, K, True, 1.0, act)
  check_flips(dev.topk_idx, own.topk_idx, lg_dev, lg_own, own.scores_for_choice, act)
  # one token's last expert replaced by its lowest-ranked one
  bad = dev.topk_idx.copy()
  worst = int(np.argmin(own.scores_for_choice[3]))
  bad[3, K - 1] = worst
  with pytest.raises(AssertionError, match="token 3 position 7"):
    check_flips(bad, own.topk_idx, lg_dev, lg_own, own.scores_for_choice, act)


def test_the_bound_follows_the_gate_slope():
  """The Lipschitz bounds used: the sigmoid's slope is at most 1/4 (at 0); a
  softmax component moves by at most 1/2 under a max-norm logit change."""
  x = np.linspace(-8, 8, 4001)
  s = 1 / (1 + np.exp(-x))
  assert np.max(np.diff(s) / np.diff(x)) <= gate_lipschitz("sigmoid") + 1e-9
  rng = np.random.default_rng(9)
  for _ in range(200):
    z = rng.standard_normal(16) * 3
    d = rng.uniform(-1, 1, 16) * 1e-4
    p = np.exp(z - z.max()) / np.exp(z - z.max()).sum()
    q = np.exp(z + d - (z + d).max()) / np.exp(z + d - (z + d).max()).sum()
    assert np.max(np.abs(q - p)) <= gate_lipschitz("softmax") * np.max(np.abs(d)) * (1 + 1e-3)


def _mx8_layer_stages(seed=3, t=64, h=128, lat=64, inter=64, e=32, k=4, start=8, L=8):
  """A small local-shard layer run through the oracle with MXFP8 activations
  in both expert GEMMs, staged the way the device layer returns its stages."""
  from lmoe.config import LatentMoEConfig
  rng = np.random.default_rng(seed)
  cfg = LatentMoEConfig(hidden_size=h, latent_size=lat, intermediate_size=inter, num_experts=e, top_k=k,
                        num_shared_experts=0)
  bf = lambda *s: O.bf16_round(rng.standard_normal(s) * 0.1)
  w = {"router_weight": bf(h, e), "e_score_correction_bias": np.zeros(e, np.float32), "down_proj": bf(h, lat),
       "up_proj": bf(lat, h), "norm_scale": O.bf16_round(1 + rng.standard_normal(lat) * 0.1)}
  ex = {"gu_packed": rng.integers(0, 256, (L + 1, 2 * inter, lat // 2), dtype=np.uint8),
        "gu_scale": rng.integers(120, 126, (L + 1, 2 * inter, lat // 32), dtype=np.uint8),
        "down_packed": rng.integers(0, 256, (L + 1, lat, inter // 2), dtype=np.uint8),
        "down_scale": rng.integers(120, 126, (L + 1, lat, inter // 32), dtype=np.uint8)}
  for key in ("gu_packed", "down_packed"):
    ex[key][L] = 0  # the padding expert: zero codes
  hidden = O.bf16_round(rng.standard_normal((t, h)))
  x = O.matmul(hidden, w["down_proj"], "bf16")
  logits = O.matmul(hidden, w["router_weight"], "f32")
  r = O.router_from_logits(logits, w["e_score_correction_bias"], k, True, 1.0, "sigmoid", "bf16")
  d = O.filter_and_pad_to_shard_jittable(r.topk_idx, r.topk_weight, x, k, e, start, L, 2.0)
  q, s = O.quantize_mxfp8(d.sorted_tokens)
  act = O.ragged_dot_mxfp8_mxfp4(q, s, ex["gu_packed"], ex["gu_scale"], d.group_sizes, "bf16", situ=(4.0, 25.0))
  q, s = O.quantize_mxfp8(act)
  shard = O.ragged_dot_mxfp8_mxfp4(q, s, ex["down_packed"], ex["down_scale"], d.group_sizes, "bf16")
  routed = O.combine_shard_contribution(np.zeros((t, lat), np.float32), shard, d.padded_token_idx,
                                        d.padded_combine_weight, "bf16", "bf16", "bf16")
  out = O.matmul(O.rms_norm(routed, w["norm_scale"], cfg.rms_norm_eps, "bf16"), w["up_proj"], "bf16")
  st = {"x": x, "router_logits": logits, "topk_idx": r.topk_idx, "topk_weight": r.topk_weight, "dispatch": d,
        "act": act, "shard_out": shard, "routed_out": routed}
  return hidden, w, ex, cfg, start, L, out, st


def test_scaled_layer_checker_accepts_the_oracle_and_rejects_a_planted_error():
  """The scaled-MFMA layer check (used on the device's stages) passes the
  oracle's own MXFP8 pipeline and fails when one row of one stage is off."""
  from _layer_check import check_single_shard_mx8
  hidden, w, ex, cfg, start, L, out, st = _mx8_layer_stages()
  assert int(st["dispatch"].group_sizes[:L].sum()) > 0  # the shard receives rows
  errs = check_single_shard_mx8("oracle as device", hidden, w, ex, cfg, start, L, 2.0, out, st)
  assert max(errs.values()) == 0.0
  row = int(np.argmax(np.abs(st["act"]).sum(axis=1)))
  bad = dict(st, act=st["act"].copy())
  bad["act"][row] *= 1.1
  with pytest.raises(AssertionError, match="act"):
    check_single_shard_mx8("planted", hidden, w, ex, cfg, start, L, 2.0, out, bad)
  bad = dict(st, topk_idx=st["topk_idx"].copy())
  bad["topk_idx"][0, 0] = (bad["topk_idx"][0, 0] + 1) % cfg.num_experts
  with pytest.raises(AssertionError, match="routing"):
    check_single_shard_mx8("planted", hidden, w, ex, cfg, start, L, 2.0, out, bad)
