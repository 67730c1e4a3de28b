"""Pins the oracle's routing / dispatch / combine restatement.

Restates the reference's CPU unit tests (05_ragged_dot_on_tpu/
test_sharded_routing_local.py:62-412) and in-module self-checks
(kimi_k3_latent_moe_reference.py:438-471, 880-939, 1190-1379, 1531-1674) as
pytest.  Literal inputs transfer verbatim; random inputs come from numpy
generators (JAX PRNG streams are not reproducible here), and every check is
against an independent brute force or a closed form, never against the
function's own formula.
"""
import numpy as np
import pytest

from lmoe.config import LatentMoEConfig
from oracle import lmoe_oracle as O


def _toy_shard_config(top_k=4, num_experts=32):
  """test_sharded_routing_local.py:51-57."""
  return LatentMoEConfig(hidden_size=64, latent_size=32, intermediate_size=48,
                         num_experts=num_experts, top_k=top_k, num_shared_experts=1)


def _dispatch(topk_idx, topk_w, x, cfg, start, L, cf, tile=1):
  return O.filter_and_pad_to_shard(topk_idx, topk_w, x, cfg.top_k, cfg.num_experts, start, L,
                                   capacity_factor=cf, tile_size=tile)


def _route(hidden, x, router_weight, bias, cfg, start, L, cf, tile=O.MOSAIC_TILE_SIZE):
  r, _ = O.router_gate(hidden, router_weight, bias, cfg, weight_dtype="f32")
  return r, _dispatch(r.topk_idx, r.topk_weight, x, cfg, start, L, cf, tile)


def test_empty_shard():
  """test_sharded_routing_local.py:62-99 (literal topk_idx)."""
  cfg = _toy_shard_config(top_k=2, num_experts=8)
  topk_idx = np.array([[0, 1], [1, 2], [6, 7], [7, 0], [2, 3]], np.int32)
  w = np.full((5, 2), 0.5, np.float32)
  x = np.random.default_rng(0).standard_normal((5, cfg.latent_size)).astype(np.float32)
  d = _dispatch(topk_idx, w, x, cfg, 4, 2, 4.0)
  assert d.per_expert_counts.sum() == 0 and d.valid_mask.sum() == 0
  assert np.all(d.sorted_tokens == 0) and np.all(d.padded_combine_weight == 0)
  assert np.all(d.padded_token_idx == -1)
  assert d.group_sizes.tolist() == [0, 0, len(d.valid_mask)]


def test_extreme_skew_concentration():
  """test_sharded_routing_local.py:102-125."""
  cfg = _toy_shard_config(top_k=1, num_experts=16)
  topk_idx = np.full((50, 1), 5, np.int32)
  w = np.full((50, 1), 0.7, np.float32)
  x = np.random.default_rng(1).standard_normal((50, cfg.latent_size)).astype(np.float32)
  d = _dispatch(topk_idx, w, x, cfg, 3, 5, 4.0)
  assert d.per_expert_counts.tolist() == [0, 0, 50, 0, 0]
  assert d.valid_mask.sum() == 50
  assert d.padded_token_idx[:50].tolist() == list(range(50))  # stable


def test_capacity_overflow_matches_python_sorted():
  """test_sharded_routing_local.py:128-167: truncation drops exactly the tail of
  a Python stable ``sorted()`` order."""
  cfg = _toy_shard_config(top_k=1, num_experts=8)
  rng = np.random.default_rng(2)
  topk_idx = rng.integers(0, 4, (20, 1)).astype(np.int32)
  w = np.full((20, 1), 0.3, np.float32)
  x = rng.standard_normal((20, cfg.latent_size)).astype(np.float32)
  d = _dispatch(topk_idx, w, x, cfg, 0, 4, 0.1)
  m_padded = int(d.group_sizes.sum())
  keep = int(d.valid_mask.sum())
  assert keep < 20 and keep == m_padded == 1
  hits = sorted(enumerate(topk_idx.reshape(-1).tolist()), key=lambda p: p[1])
  assert d.padded_token_idx[:keep].tolist() == [t for t, _ in hits[:m_padded]]


def test_padding_does_not_contaminate():
  """test_sharded_routing_local.py:170-194: non-zero padding rows with weight 0
  add nothing."""
  shard_out = np.random.default_rng(3).standard_normal((6, 8)).astype(np.float32)
  idx = np.array([0, 1, 2, 3, -1, -1], np.int32)
  w = np.array([0.5, 0.5, 0.5, 0.5, 0.0, 0.0], np.float32)
  out = O.combine_shard_contribution(np.zeros((4, 8), np.float32), shard_out, idx, w,
                                     "f32", "f32", "f32")
  assert np.max(np.abs(out - shard_out[:4] * 0.5)) < 1e-6


def test_top_k_16():
  """test_sharded_routing_local.py:197-229."""
  cfg = _toy_shard_config(top_k=16, num_experts=64)
  rng = np.random.default_rng(4)
  router_weight = (rng.standard_normal((64, 64)) * 0.02).astype(np.float32)
  hidden = rng.standard_normal((128, 64)).astype(np.float32)
  r, d = _route(hidden, hidden, router_weight, np.zeros(64, np.float32), cfg, 10, 16, 4.0)
  assert d.sorted_tokens.shape[1] == 64
  assert d.per_expert_counts.sum() == d.valid_mask.sum() <= d.sorted_tokens.shape[0]
  # brute-force count of in-shard picks
  assert d.per_expert_counts.sum() == ((r.topk_idx >= 10) & (r.topk_idx < 26)).sum()


def test_global_to_local_boundary():
  """test_sharded_routing_local.py:232-266 (literal ids 4/5/8/9)."""
  cfg = _toy_shard_config(top_k=1, num_experts=20)
  topk_idx = np.array([[4], [5], [8], [9]], np.int32)
  w = np.array([[0.1], [0.2], [0.3], [0.4]], np.float32)
  x = np.random.default_rng(5).standard_normal((4, cfg.latent_size)).astype(np.float32)
  d = _dispatch(topk_idx, w, x, cfg, 5, 4, 4.0)
  keep = int(d.valid_mask.sum())
  assert sorted(d.padded_token_idx[:keep].tolist()) == [1, 2]
  assert d.per_expert_counts.tolist() == [1, 0, 0, 1]
  assert d.padded_combine_weight[:keep].tolist() == [np.float32(0.2), np.float32(0.3)]


def test_first_and_last_shard():
  """test_sharded_routing_local.py:269-305."""
  cfg = _toy_shard_config(top_k=2, num_experts=24)
  rng = np.random.default_rng(6)
  router_weight = (rng.standard_normal((64, 24)) * 0.02).astype(np.float32)
  hidden = rng.standard_normal((64, 64)).astype(np.float32)
  for shard in (0, 3):
    r, d = _route(hidden, hidden, router_weight, np.zeros(24, np.float32), cfg, shard * 6, 6, 4.0)
    assert d.valid_mask.sum() == d.per_expert_counts.sum()
    assert d.per_expert_counts.sum() == ((r.topk_idx >= shard * 6) & (r.topk_idx < shard * 6 + 6)).sum()


def test_batch_seq_invariance():
  """test_sharded_routing_local.py:308-339: only num_tokens matters; a
  (batch, seq) reshape of the same tokens changes nothing."""
  cfg = _toy_shard_config(top_k=4, num_experts=16)
  rng = np.random.default_rng(7)
  router_weight = (rng.standard_normal((64, 16)) * 0.02).astype(np.float32)
  hidden = rng.standard_normal((4, 8, 64)).astype(np.float32)
  a = _route(hidden.reshape(32, 64), hidden.reshape(32, 64), router_weight,
             np.zeros(16, np.float32), cfg, 0, 8, 4.0)[1]
  b = _route(hidden.reshape(-1, 64), hidden.reshape(-1, 64), router_weight,
             np.zeros(16, np.float32), cfg, 0, 8, 4.0)[1]
  for x, y in zip(a, b):
    assert np.array_equal(x, y)


def test_dtype_no_silent_promotion():
  """test_sharded_routing_local.py:342-392: bf16 in -> bf16-exact out, including
  the empty-group branch of the shard FFN."""
  cfg = _toy_shard_config(top_k=2, num_experts=8)
  x = O.bf16_round(np.random.default_rng(8).standard_normal((6, cfg.latent_size)))
  d = _dispatch(np.full((6, 2), 5, np.int32), O.bf16_round(np.full((6, 2), 0.5)), x, cfg, 0, 2, 4.0)
  assert np.array_equal(d.sorted_tokens, O.bf16_round(d.sorted_tokens))
  gs = np.array([0, 0, 3], np.int32)
  z = np.zeros((3, cfg.latent_size, cfg.intermediate_size), np.float32)
  zd = np.zeros((3, cfg.intermediate_size, cfg.latent_size), np.float32)
  out = O.local_shard_expert_ffn(np.zeros((3, cfg.latent_size), np.float32), z, z, zd, gs, cfg, "bf16")
  assert out.shape == (3, cfg.latent_size) and np.all(out == 0)


def _init_weights(cfg, rng):
  """ref.py:255-283 shapes, N(0, 0.02^2), zero bias, unit norm scale (numpy PRNG)."""
  si = cfg.intermediate_size * cfg.num_shared_experts
  n = lambda *s: (rng.standard_normal(s) * 0.02).astype(np.float32)
  return {
      "router_weight": n(cfg.hidden_size, cfg.num_experts),
      "e_score_correction_bias": np.zeros(cfg.num_experts, np.float32),
      "down_proj": n(cfg.hidden_size, cfg.latent_size),
      "up_proj": n(cfg.latent_size, cfg.hidden_size),
      "expert_gate": n(cfg.num_experts, cfg.latent_size, cfg.intermediate_size),
      "expert_up": n(cfg.num_experts, cfg.latent_size, cfg.intermediate_size),
      "expert_down": n(cfg.num_experts, cfg.intermediate_size, cfg.latent_size),
      "norm_scale": np.ones(cfg.latent_size, np.float32),
      "shared_gate": n(cfg.hidden_size, si),
      "shared_up": n(cfg.hidden_size, si),
      "shared_down": n(si, cfg.hidden_size),
  }


@pytest.mark.parametrize("seed,num_tokens,global_e,local_e,top_k", [
    (0, 32, 16, 4, 2), (1, 96, 32, 8, 4), (2, 64, 48, 16, 6), (3, 200, 64, 8, 16)])
def test_sharded_sum_matches_unsharded(seed, num_tokens, global_e, local_e, top_k):
  """ref.py:1531-1674 over the four configs of test_sharded_routing_local.py:395-412:
  route+filter+per-shard FFN+combine summed over all shards == unsharded forward."""
  cfg = _toy_shard_config(top_k=top_k, num_experts=global_e)
  rng = np.random.default_rng(seed)
  w = _init_weights(cfg, rng)
  hidden = rng.standard_normal((num_tokens, cfg.hidden_size)).astype(np.float32)
  reference, _ = O.latent_moe_forward(hidden, w, cfg, "f32")
  x = O.matmul(hidden, w["down_proj"], "f32")
  routed = np.zeros((num_tokens, cfg.latent_size), np.float32)
  total_valid = 0
  for s in range(global_e // local_e):
    start = s * local_e
    r, d = _route(hidden, x, w["router_weight"], w["e_score_correction_bias"], cfg, start, local_e,
                  4.0, tile=1)
    total_valid += int(d.valid_mask.sum())
    pad = lambda a: np.concatenate([a[start:start + local_e], np.zeros_like(a[:1])])
    out = O.local_shard_expert_ffn(d.sorted_tokens, pad(w["expert_gate"]), pad(w["expert_up"]),
                                   pad(w["expert_down"]), d.group_sizes, cfg, "f32")
    routed = O.combine_shard_contribution(routed, out, d.padded_token_idx, d.padded_combine_weight,
                                          "f32", "f32", "f32")
  assert total_valid == num_tokens * top_k
  normed = O.rms_norm(routed, w["norm_scale"], cfg.rms_norm_eps, "f32")
  final = O.matmul(normed, w["up_proj"], "f32") + O.situ_glu_mlp(
      hidden, w["shared_gate"], w["shared_up"], w["shared_down"], 4.0, 25.0, "f32")
  assert np.max(np.abs(final - reference)) < 1e-4


def test_route_and_filter_brute_force_real_scale():
  """ref.py:1190-1379: E=896, k=16, local_expert_start=137, L=64; counts vs a
  nested loop, gather vs x[idx], weights vs the (token, slot) they came from,
  forced overflow (cf=0.05, tile=1) vs Python stable sorted()."""
  from lmoe.config import kimi_k3_config
  cfg = kimi_k3_config()
  rng = np.random.default_rng(0)
  hidden = rng.standard_normal((256, cfg.hidden_size)).astype(np.float32)
  router_weight = (rng.standard_normal((cfg.hidden_size, 896)) * 0.02).astype(np.float32)
  start, L = 137, 64
  r, d = _route(hidden, hidden, router_weight, np.zeros(896, np.float32), cfg, start, L, 4.0)
  ti = r.topk_idx
  ref_counts = [0] * L
  for tok in range(ti.shape[0]):
    for slot in range(ti.shape[1]):
      g = int(ti[tok, slot])
      if start <= g < start + L:
        ref_counts[g - start] += 1
  assert d.per_expert_counts.tolist() == ref_counts
  nv = int(d.valid_mask.sum())
  assert np.array_equal(d.sorted_tokens[:nv], hidden[d.padded_token_idx[:nv]])
  # each kept row's weight is its own (token, slot) weight, found by expert id
  row_expert = np.repeat(np.arange(L), d.per_expert_counts) + start
  for row in range(nv):
    tok = d.padded_token_idx[row]
    slot = int(np.nonzero(ti[tok] == row_expert[row])[0][0])
    assert d.padded_combine_weight[row] == r.topk_weight[tok, slot]
  # forced overflow
  d2 = _dispatch(ti, r.topk_weight, hidden, cfg, start, L, 0.05, tile=1)
  m_padded = int(d2.group_sizes.sum())
  hits = sorted([(int(g) - start, tok) for tok in range(ti.shape[0]) for g in ti[tok]
                 if start <= g < start + L], key=lambda p: p[0])
  kept = hits[:m_padded]
  assert len(hits) > m_padded
  assert int(d2.valid_mask.sum()) == len(kept)
  assert d2.padded_token_idx[:len(kept)].tolist() == [t for _, t in kept]
  assert d2.per_expert_counts.tolist() == np.bincount([l for l, _ in kept], minlength=L).tolist()


@pytest.mark.parametrize("name,num_tokens,global_e,start,L,cf", [
    ("standard", 64, 32, 5, 8, 2.0), ("overflow", 64, 32, 5, 8, 0.05), ("decode_scale", 1, 32, 5, 8, 2.0)])
def test_eager_equals_jittable(name, num_tokens, global_e, start, L, cf):
  """ref.py:880-939: the sentinel-keyed fixed-shape dispatch is bit-identical to
  the filter-first eager dispatch (standard, forced overflow, decode T=1)."""
  cfg = _toy_shard_config(top_k=2, num_experts=global_e)
  rng = np.random.default_rng({"standard": 11, "overflow": 12, "decode_scale": 13}[name])
  ti = rng.integers(0, global_e, (num_tokens, 2)).astype(np.int32)
  tw = rng.uniform(size=(num_tokens, 2)).astype(np.float32)
  x = O.bf16_round(rng.standard_normal((num_tokens, 32)))
  a = O.filter_and_pad_to_shard(ti, tw, x, 2, global_e, start, L, cf)
  b = O.filter_and_pad_to_shard_jittable(ti, tw, x, 2, global_e, start, L, cf)
  for u, v in zip(a, b):
    assert u.shape == v.shape and np.array_equal(u, v)


def test_dispatch_roundtrip_identity():
  """ref.py:438-471: dispatch then inverse permutation with an identity expert
  returns every token's vector to each of its slots."""
  rng = np.random.default_rng(9)
  x = rng.standard_normal((20, 32)).astype(np.float32)
  ti = O.top_k(rng.uniform(size=(20, 8)), 2)
  order, sorted_tokens, gs = O.unsharded_dispatch(ti, x, 8)
  _, unsorted = O.unsharded_combine(sorted_tokens, order, np.ones((20, 2), np.float32), 20, 2, "f32")
  assert np.max(np.abs(unsorted - x[:, None, :])) < 1e-6
  assert gs.sum() == 40 and np.array_equal(gs, np.bincount(ti.reshape(-1), minlength=8))


def test_slot_pos_is_inverse_permutation():
  """slot_pos (not a reference output) inverts the jittable dispatch order."""
  rng = np.random.default_rng(10)
  ti = np.stack([rng.permutation(40)[:6] for _ in range(50)]).astype(np.int32)
  tw = rng.uniform(size=(50, 6)).astype(np.float32)
  d, slot_pos = O.filter_and_pad_to_shard_jittable(ti, tw, np.zeros((50, 4), np.float32), 6, 40,
                                                   8, 16, 1.0, tile_size=16, return_slot_pos=True)
  for s, p in enumerate(slot_pos):
    t, j = divmod(s, 6)
    if p >= 0:
      assert d.padded_token_idx[p] == t and d.padded_combine_weight[p] == tw[t, j]
      assert int(ti[t, j]) - 8 == np.searchsorted(np.cumsum(d.group_sizes), p, side="right")
  assert (slot_pos >= 0).sum() == d.valid_mask.sum()


def test_combine_scatter_add_rounds_each_add_in_order():
  """Scatter-add in bf16 rounds after every add, in ascending row order:
  1 + 5*2^-10 + 5*2^-10 as two rounded adds is 1 + 2^-6, while the f32 sum
  rounded once would be 1 + 2^-7."""
  shard = np.array([[5 * 2.0 ** -10], [5 * 2.0 ** -10]], np.float32)
  out = O.combine_shard_contribution(np.ones((1, 1), np.float32), shard, np.array([0, 0]),
                                     np.ones(2, np.float32), "bf16", "bf16", "bf16")
  assert out[0, 0] == np.float32(1 + 2.0 ** -6)
  assert O.bf16_round(np.float32(1 + 10 * 2.0 ** -10)) == np.float32(1 + 2.0 ** -7)


@pytest.mark.parametrize("t,k,want", [(128, 16, 384), (2048, 16, 4736), (4096, 16, 9472)])
def test_compute_m_padded_reference_table(t, k, want):
  """The reference's Stage C table (expert_ffn_roofline.py:42-47, a 64-expert
  shard of 896, top-16, capacity factor 2) at its prefill token sweep
  (rd.py:1843: 128, 2048, 4096 tokens)."""
  assert O.compute_m_padded(t, k, 896, 64, 2.0) == want


@pytest.mark.parametrize("seed,num_tokens,global_e,local_e,top_k", [(0, 32, 16, 4, 2), (3, 96, 32, 8, 8)])
def test_single_shard_forward_against_unsharded(seed, num_tokens, global_e, local_e, top_k):
  """One shard holding every expert reproduces ``latent_moe_forward`` stage by
  stage (f32; only the combine's summation order differs), and the routed
  outputs of all shards of a split sum to the unsharded routed output."""
  cfg = _toy_shard_config(top_k=top_k, num_experts=global_e)
  rng = np.random.default_rng(seed)
  w = _init_weights(cfg, rng)
  hidden = rng.standard_normal((num_tokens, cfg.hidden_size)).astype(np.float32)
  want, inter = O.latent_moe_forward(hidden, w, cfg, "f32")
  pad = lambda a, s, n: np.concatenate([a[s:s + n], np.zeros_like(a[:1])])
  shard = lambda s, n: [pad(w[k], s, n) for k in ("expert_gate", "expert_up", "expert_down")]
  got, st = O.single_shard_forward(hidden, w, *shard(0, global_e), cfg, "f32", 0, global_e,
                                   capacity_factor=float(global_e))
  assert np.array_equal(st["x"], inter["latent_projection"])
  assert np.array_equal(st["router_logits"], inter["router_logits"])
  assert np.array_equal(st["topk_idx"], inter["topk_indices"])
  assert np.array_equal(st["topk_weight"], inter["topk_weights"])
  assert int(st["dispatch"].valid_mask.sum()) == num_tokens * top_k
  assert np.max(np.abs(st["routed_out"] - inter["routed_output_after_combine"])) < 1e-5
  assert np.max(np.abs(got - want)) < 1e-4
  routed = sum(O.single_shard_forward(hidden, w, *shard(s, local_e), cfg, "f32", s, local_e,
                                      capacity_factor=float(global_e // local_e), include_shared=False)[1]["routed_out"]
               for s in range(0, global_e, local_e))
  assert np.max(np.abs(routed - inter["routed_output_after_combine"])) < 1e-5
