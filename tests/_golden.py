"""Loader for the committed golden bundles (tests/golden/golden_bundle_*).

The bundles are copies of the reference's
06_kimi_k3_golden_validation/golden_bundle_*/{inputs,weights,golden_outputs}.npz
(+ config.json, metadata.json); provenance and sha256 in tests/golden/SHA256SUMS.
They were produced by the official PyTorch KimiSparseMoeBlock at reduced scale.
"""
import json
import os

import numpy as np

GOLDEN_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
# all six bundles the reference holds: 64/32/48 and 256/128/128 (T = 20),
# 256/128/128 (T = 64), each in fp32 and bf16
BUNDLES = ("golden_bundle_small", "golden_bundle_small_bf16",
           "golden_bundle_mosaic_fp32", "golden_bundle_mosaic_bf16",
           "golden_bundle_mosaic_fp32_n64", "golden_bundle_mosaic_bf16_n64")

# test_jax_reference_against_pytorch_golden.py:94-97
TOLERANCES = {"f32": (1e-4, 1e-3), "bf16": (1e-3, 1e-3)}

# The reference documents that every one of its implementations (xla, mosaic,
# mosaic_tpu_v2) misses the bf16 tolerance on the 256/128/128 bundles on the same
# four stages by one bf16 ulp, with these max abs diffs, on the n=20 and n=64
# bundles alike (README.md:175-195).  A faithful restatement shows the same
# residual, no larger.
_MOSAIC_BF16_RESIDUAL = {
    "expert_up_output": 1.953125e-3,
    "up_projection_output": 7.8125e-3,
    "final_output": 7.8125e-3,
    "normalized_output": 1.5625e-2,
}
KNOWN_RESIDUALS = {
    "golden_bundle_mosaic_bf16": _MOSAIC_BF16_RESIDUAL,
    "golden_bundle_mosaic_bf16_n64": _MOSAIC_BF16_RESIDUAL,
}


def load(name):
  from lmoe.config import config_from_official, weights_from_official_state_dict
  d = os.path.join(GOLDEN_DIR, name)
  inputs = np.load(os.path.join(d, "inputs.npz"))
  weights = np.load(os.path.join(d, "weights.npz"))
  outputs = np.load(os.path.join(d, "golden_outputs.npz"))
  with open(os.path.join(d, "config.json")) as f:
    official = json.load(f)
  with open(os.path.join(d, "metadata.json")) as f:
    meta = json.load(f)
  config = config_from_official(official)
  dtype = "bf16" if meta["dtype"].endswith("bfloat16") else "f32"
  w = weights_from_official_state_dict({k: weights[k] for k in weights.files}, config)
  hidden = inputs["hidden_states"][0]
  return config, dtype, hidden, w, {k: outputs[k] for k in outputs.files}


def canonical_order(token_ids, group_sizes):
  """(expert_id, token_id) re-sort key for per-dispatch-slot arrays,
  test_jax_reference_against_pytorch_golden.py:278-289."""
  expert_of_slot = np.repeat(np.arange(len(group_sizes)), group_sizes)
  return np.lexsort((token_ids, expert_of_slot))


def compare_stages(golden, ours, config, dtype, check):
  """Stage-by-stage comparison with the reference's canonicalisation
  (test_jax_reference_against_pytorch_golden.py:307-445).  ``ours`` holds the
  18 intermediates; ``check(name, golden, ours, exact)`` asserts."""
  k = config.top_k
  check("group_sizes", golden["group_sizes"], np.asarray(ours["group_sizes"]), True)
  g_idx, j_idx = golden["topk_indices"], np.asarray(ours["topk_indices"])
  g_ord, j_ord = np.argsort(g_idx, axis=-1), np.argsort(j_idx, axis=-1)
  check("topk_indices", np.take_along_axis(g_idx, g_ord, -1), np.take_along_axis(j_idx, j_ord, -1), True)
  check("topk_weights", np.take_along_axis(golden["topk_weights"], g_ord, -1),
        np.take_along_axis(np.asarray(ours["topk_weights"]), j_ord, -1), False)
  for key in ("router_logits", "router_scores_before_bias", "router_scores_for_choice",
              "latent_projection"):
    check(key, golden[key], np.asarray(ours[key]), False)
  g_tok = golden["sorted_token_indices"] // k
  j_tok = np.asarray(ours["sorted_token_indices"]) // k
  g_can = canonical_order(g_tok, golden["group_sizes"])
  j_can = canonical_order(j_tok, np.asarray(ours["group_sizes"]))
  check("sorted_token_indices", g_tok[g_can], j_tok[j_can], True)
  for key in ("expert_gate_output", "expert_up_output", "situ_output", "expert_down_output"):
    check(key, golden[key][g_can], np.asarray(ours[key])[j_can], False)
  lat = config.latent_size
  gb = golden["routed_output_before_combine"].reshape(-1, k, lat)
  jb = np.asarray(ours["routed_output_before_combine"]).reshape(-1, k, lat)
  check("routed_output_before_combine", np.take_along_axis(gb, g_ord[:, :, None], 1),
        np.take_along_axis(jb, j_ord[:, :, None], 1), False)
  for key in ("routed_output_after_combine", "normalized_output", "up_projection_output"):
    check(key, golden[key], np.asarray(ours[key]), False)
  h = config.hidden_size
  check("shared_expert_output", golden["shared_expert_output"].reshape(-1, h),
        np.asarray(ours["shared_expert_output"]), False)
  check("final_output", golden["final_output"].reshape(-1, h), np.asarray(ours["final_output"]), False)
