"""Whole-layer parity checks shared by the GPU forward tests.

The device computes the router logits and the latent projection with its own
GEMM summation order, so its logits may differ from the oracle's in the last
f32 bits and, rarely, flip a near-tied top-k choice.  Rather than skipping the
numeric checks when that happens, the layer is checked in two parts, both
always asserted:

1. the device's logits and latent projection against the oracle's own (f32
   1e-5 / bf16 2e-2 max-relative), and its routing against the oracle's
   routing of the oracle's own logits (agreement reported; every token that
   differs must be a near tie that the measured logit error explains);
2. the oracle's forward run on the device's logits and latent projection:
   routing ids and weights bit-exact, all dispatch outputs bit-exact, and
   every later stage (expert FFN, combine, norm, up-projection, final) within
   the bf16 / f32 bar.
"""
import numpy as np

from _util import banner, max_rel, to_np
from oracle import lmoe_oracle as O


def _tol(dtype):
  return 1e-5 if dtype == "f32" else 2e-2


def gate_lipschitz(act):
  """Largest change of one gate score per unit change of the logits in the
  max-norm: sigmoid' <= 1/4; a softmax component moves by at most
  p (1 - p) + p (1 - p) <= 1/2 (its own logit and all the others)."""
  return 0.25 if act == "sigmoid" else 0.5


def check_flips(idx_dev, idx_own, lg_dev, lg_own, choice_own, act):
  """Tokens whose top-k on the device's logits differs from the oracle's on
  its own logits (another f32 GEMM summation order) must be near ties.  At
  the first top-k position j where the two differ, the oracle took expert a
  and the device expert b from the same remaining set, so with every
  selection key (gate score + bias) moved by at most eta between the two
  logit rows, key(a) - key(b) <= 2 eta, where eta = L * max_e |dlogit| (L the
  gate's Lipschitz bound) plus the keys' f32 rounding.  A token routed
  differently with a wider gap is a routing error, however few there are.
  Returns the number of tokens that differ."""
  lip = gate_lipschitz(act)
  rows = np.nonzero(np.any(idx_dev != idx_own, axis=1))[0]
  for t in rows:
    j = int(np.argmax(idx_dev[t] != idx_own[t]))
    a, b = int(idx_own[t, j]), int(idx_dev[t, j])
    dlog = float(np.max(np.abs(np.asarray(lg_dev[t], np.float64) - np.asarray(lg_own[t], np.float64))))
    # each f32 key is rounded twice (score, then score + bias) on each side
    eta = lip * dlog + 2.0 ** -21 * max(1.0, float(np.max(np.abs(choice_own[t]))))
    gap = float(choice_own[t, a]) - float(choice_own[t, b])
    assert 0.0 <= gap <= 2.0 * eta, (f"token {t} position {j}: oracle expert {a}, device expert {b}, key gap "
                                     f"{gap:.3e} > 2 x {eta:.3e} (logits moved {dlog:.3e})")
  return len(rows)


def check_single_shard(name, hidden, w, gate, up, down, cfg, dtype, start, L, cf, include_shared, out, st,
                       act="sigmoid"):
  """``out`` / ``st``: the device forward's output and stage dict (keys
  x, router_logits, topk_idx, topk_weight, dispatch, shard_out, routed_out);
  ``gate``/``up``/``down``: (L+1, in, out) f32 arrays of the shard."""
  tol = _tol(dtype)
  own_final, own = O.single_shard_forward(hidden, w, gate, up, down, cfg, dtype, start, L, cf, act=act,
                                          include_shared=include_shared)
  x_dev, lg_dev = to_np(st["x"]), to_np(st["router_logits"])
  err_x = max_rel(x_dev, own["x"])
  err_lg = max_rel(lg_dev, own["router_logits"])
  idx_dev = to_np(st["topk_idx"])
  agree = np.all(idx_dev == own["topk_idx"], axis=1)
  ref, rs = O.single_shard_forward(hidden, w, gate, up, down, cfg, dtype, start, L, cf, act=act,
                                   include_shared=include_shared, logits=lg_dev, x=x_dev)
  errs = {
      "shard_out": max_rel(to_np(st["shard_out"]), rs["shard_out"]),
      "routed_out": max_rel(to_np(st["routed_out"]), rs["routed_out"]),
      "final": max_rel(to_np(out), ref),
  }
  # rows whose routing agrees with the oracle's own logits: the device output
  # against the fully independent oracle forward
  out_np = to_np(out)
  err_own = max_rel(out_np[agree], own_final[agree]) if agree.any() else 0.0
  banner(f"{name}: x {err_x:.2e} logits {err_lg:.2e} routing agreement {agree.mean():.5f} "
         f"({(~agree).sum()} tokens differ on own logits); on device logits: "
         + " ".join(f"{k} {v:.2e}" for k, v in errs.items()) + f"; final vs own oracle (agreeing rows) {err_own:.2e}")
  assert err_x <= 2e-2, err_x
  assert err_lg <= 1e-5, err_lg
  check_flips(idx_dev, own["topk_idx"], lg_dev, own["router_logits"], own["router_scores_for_choice"], act)
  assert np.array_equal(idx_dev, rs["topk_idx"]), "routing differs on identical logits"
  assert np.array_equal(to_np(st["topk_weight"]), rs["topk_weight"]), "routing weights differ on identical logits"
  d = rs["dispatch"]
  for field, a, b in zip(d._fields, st["dispatch"][:6], d):
    assert np.array_equal(to_np(a), b), f"dispatch {field}"
  for k, v in errs.items():
    assert v <= tol, (k, v)
  assert err_own <= tol, err_own
  return errs


def _np(a):
  return to_np(a) if hasattr(a, "detach") else np.asarray(a)


def check_single_shard_mx8(name, hidden, w, experts, cfg, start, L, cf, out, st, act="sigmoid"):
  """The bf16 layer with ``mxfp4_mode="scaled_mfma"``: both expert GEMMs take
  MXFP8 activations (E4M3 + E8M0 per 32, quantised on the device) x MXFP4
  weights.  The oracle runs each stage on the device's own input to it:
  routing and dispatch from the device's logits and latent rows (bit-exact);
  gate/up + SiTU on the dispatched rows and the down projection on the
  device's SiTU output through the oracle's MXFP8 x MXFP4 product (the
  device's quantiser is bit-exact against the oracle's, the product exact up
  to the block-scaled instruction's accumulation); the combine on the
  device's shard output and the RMSNorm + up-projection on the device's
  combined rows.  Every stage within the bf16 bar.  ``experts``: numpy
  checkpoint-layout gu/down packed codes and scales of the L + 1 experts;
  ``out`` / ``st`` as in ``check_single_shard`` (torch or numpy arrays)."""
  tol = 2e-2
  x_dev, lg_dev = _np(st["x"]), _np(st["router_logits"])
  r = O.router_from_logits(lg_dev, w["e_score_correction_bias"], cfg.top_k, cfg.moe_renormalize,
                           cfg.routed_scaling_factor, act, "bf16")
  assert np.array_equal(_np(st["topk_idx"]), r.topk_idx), "routing differs on identical logits"
  assert np.array_equal(_np(st["topk_weight"]), r.topk_weight), "routing weights differ on identical logits"
  d = O.filter_and_pad_to_shard_jittable(r.topk_idx, r.topk_weight, O.cast(x_dev, "bf16"), cfg.top_k,
                                         cfg.num_experts, start, L, cf)
  for field, a, b in zip(d._fields, st["dispatch"][:6], d):
    assert np.array_equal(_np(a), b), f"dispatch {field}"
  situ = (cfg.activation_situ_beta, cfg.activation_situ_linear_beta)
  codes, scales = O.quantize_mxfp8(d.sorted_tokens)
  act_ref = O.ragged_dot_mxfp8_mxfp4(codes, scales, experts["gu_packed"], experts["gu_scale"], d.group_sizes,
                                     "bf16", situ=situ)
  act_dev = _np(st["act"])
  codes, scales = O.quantize_mxfp8(act_dev)
  shard_ref = O.ragged_dot_mxfp8_mxfp4(codes, scales, experts["down_packed"], experts["down_scale"], d.group_sizes,
                                       "bf16")
  shard_dev = _np(st["shard_out"])
  routed_ref = O.combine_shard_contribution(np.zeros((hidden.shape[0], cfg.latent_size), np.float32), shard_dev,
                                            d.padded_token_idx, d.padded_combine_weight, "bf16", "bf16", "bf16")
  routed_dev = _np(st["routed_out"])
  final_ref = O.matmul(O.rms_norm(routed_dev, w["norm_scale"], cfg.rms_norm_eps, "bf16"), w["up_proj"], "bf16")
  errs = {"act": max_rel(act_dev, act_ref), "shard_out": max_rel(shard_dev, shard_ref),
          "routed_out": max_rel(routed_dev, routed_ref), "final": max_rel(_np(out), final_ref)}
  banner(f"{name}: on the device's stage inputs: " + " ".join(f"{k} {v:.2e}" for k, v in errs.items()))
  for k, v in errs.items():
    assert v <= tol, (k, v)
  return errs


def check_unsharded(name, hidden, w, cfg, dtype, act, out, inter):
  """The unsharded forward (ref.py:330-435): ``inter`` as returned by
  ``latent_moe_forward(..., return_intermediates=True)``."""
  tol = _tol(dtype)
  own_final, own = O.latent_moe_forward(hidden, w, cfg, dtype, act=act)
  lg_dev, x_dev = to_np(inter["router_logits"]), to_np(inter["latent_projection"])
  ref, ri = O.latent_moe_forward(hidden, w, cfg, dtype, act=act, logits=lg_dev, x=x_dev)
  idx_dev = to_np(inter["topk_indices"])
  agree = np.all(idx_dev == own["topk_indices"], axis=1)
  err_lg = max_rel(lg_dev, own["router_logits"])
  err_x = max_rel(x_dev, own["latent_projection"])
  errs = {k: max_rel(to_np(inter[k]), ri[k]) for k in
          ("router_scores_before_bias", "routed_output_after_combine", "normalized_output",
           "up_projection_output", "shared_expert_output")}
  errs["final"] = max_rel(to_np(out), ref)
  banner(f"{name}: logits {err_lg:.2e} x {err_x:.2e} routing agreement {agree.mean():.5f}; on device logits: "
         + " ".join(f"{k} {v:.2e}" for k, v in errs.items()))
  assert err_lg <= 1e-5, err_lg
  assert err_x <= tol, err_x
  check_flips(idx_dev, own["topk_indices"], lg_dev, own["router_logits"], own["router_scores_for_choice"], act)
  assert np.array_equal(idx_dev, ri["topk_indices"]), "routing differs on identical logits"
  assert np.array_equal(to_np(inter["topk_weights"]), ri["topk_weights"]), "weights differ on identical logits"
  assert np.array_equal(to_np(inter["router_scores_before_bias"]), ri["router_scores_before_bias"])
  assert np.array_equal(to_np(inter["group_sizes"]), ri["group_sizes"])
  for k, v in errs.items():
    assert v <= tol, (k, v)
  return errs
