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
