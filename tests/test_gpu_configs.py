"""GPU parity at the exact sizes of the five BASELINE.json configurations.

* config 1: the reduced fp32 layer (128 tokens, 256 -> 128, 8 experts, top-2,
  one shared expert) through ``latent_moe_forward`` with the softmax gate
  (BASELINE) and the sigmoid gate (the reference's own), f32 bar 1e-5;
* config 2 is covered in test_gpu_gemm.py (``test_ragged_dot_config2_full``);
* config 3: given router logits -> top-16 of 896 -> dispatch to experts
  0..111 -> fused gate/up + SiTU -> down -> combine, at 2048 tokens, latent
  1024, intermediate 2048, 113 groups, through the reference-layout entry
  points (rd.py:726-748) and the prepared-weight layout;
* config 4: the MXFP4 matmul K = 7168, N = 2048 at M in {1, 16, 128, 1024,
  4096} through every kernel that computes it;
* config 5: the benchmarked local-shard layer at full size (4096 tokens,
  7168 -> 1024, 896 experts, top-16, experts 0..111 in MXFP4).

Routing, dispatch and the MXFP4 dequantisation are bit-exact; bf16 stages
within 2e-2 max-relative (benchmark_harness.py:192-199).
"""
import numpy as np
import pytest
import torch

from _layer_check import check_single_shard, check_unsharded
from _util import banner, max_rel, to_dev, to_np
from oracle import lmoe_oracle as O

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("act", ["softmax", "sigmoid"])
def test_config1_forward_fp32(gpu_device, act):
  from lmoe.config import LatentMoEWeights
  from lmoe.forward import latent_moe_forward
  from lmoe.workloads import make_config1
  cfg, hidden, w = make_config1()
  W = LatentMoEWeights(**{k: to_dev(v) for k, v in w.items()})
  out, inter = latent_moe_forward(to_dev(hidden), W, cfg, act=act, return_intermediates=True)
  assert out.dtype == torch.float32 and out.shape == (128, 256)
  check_unsharded(f"config 1 ({act})", hidden, w, cfg, "f32", act, out, inter)


def _config3_oracle(logits, x, gate, up, down, c):
  """Routing from the given logits, dispatch, shard FFN (gate/up rounded to
  bf16 before SiTU, rd.py:580-607 / gk.py:114-125) and the sharded combine."""
  cfg = c.config()
  r = O.router_from_logits(logits, None, c.top_k, True, 1.0, "sigmoid", "bf16")
  d = O.filter_and_pad_to_shard_jittable(r.topk_idx, r.topk_weight, x, c.top_k, c.experts, c.local_start,
                                         c.local_experts, c.capacity_factor)
  shard_out = O.local_shard_expert_ffn(d.sorted_tokens, gate, up, down, d.group_sizes, cfg, "bf16")
  routed = O.combine_shard_contribution(np.zeros((c.tokens, c.latent), np.float32), shard_out,
                                        d.padded_token_idx, d.padded_combine_weight, "bf16", "bf16", "bf16")
  return r, d, shard_out, routed


@pytest.mark.parametrize("layout", ["gkn", "gnk"])
def test_config3_fused_ffn_full_size(gpu_device, layout):
  from lmoe import ops
  from lmoe.workloads import Config3, make_config3
  c = Config3()
  cfg = c.config()
  L = c.local_experts
  banner(f"config 3 full size, {layout} weights")
  logits, x, gate, up, down = make_config3(gpu_device, c)
  idx, w = ops.router_topk_from_logits(logits, None, c.top_k, True, 1.0, "sigmoid", torch.bfloat16)
  # the reference's jittable dispatch (ref.py:754-877): a 6-tuple
  d = ops.filter_and_pad_to_shard_jittable(idx, w, x, cfg, c.local_start, L, c.capacity_factor)
  sorted_tokens, group_sizes, _, _, padded_token_idx, padded_w = d
  if layout == "gkn":
    # the reference's call: prefuse the (G, K, N) weights, fused op, down op
    shard_out = ops._local_shard_expert_ffn_ragged_dot_fused_gateup(sorted_tokens, gate, up, down,
                                                                    group_sizes, cfg, zero_group=L)
  else:
    gu_nk = ops.prefuse_gateup_weights_gnk(gate, up)
    shard_out = ops._fused_gateup_expert_ffn_from_prefused_weights(
        sorted_tokens, gu_nk, ops.to_gnk(down), group_sizes, cfg.activation_situ_beta,
        cfg.activation_situ_linear_beta, zero_group=L, rhs_layout="gnk")
  routed = ops._combine_shard_contribution(torch.zeros((c.tokens, c.latent), dtype=torch.bfloat16,
                                                       device=gpu_device), shard_out, padded_token_idx, padded_w)
  torch.cuda.synchronize()
  r, od, o_shard, o_routed = _config3_oracle(to_np(logits), to_np(x), to_np(gate), to_np(up), to_np(down), c)
  assert np.array_equal(to_np(idx), r.topk_idx)
  assert np.array_equal(to_np(w), r.topk_weight)
  for field, a, b in zip(od._fields, d, od):
    assert np.array_equal(to_np(a), b), field
  gs = od.group_sizes
  rows = int(gs[:L].sum())
  e_shard = max_rel(to_np(shard_out)[:rows], o_shard[:rows])
  e_routed = max_rel(to_np(routed), o_routed)
  banner(f"  R={rows} m_padded={gs.sum()} experts hit {(gs[:L] > 0).sum()}: shard_out {e_shard:.2e} "
         f"routed {e_routed:.2e}")
  assert e_shard <= 2e-2 and e_routed <= 2e-2
  assert not to_np(shard_out)[rows:].any()  # the padding bucket's rows are zero


CONFIG4_M = [1, 16, 128, 1024, 4096]


@pytest.fixture(scope="module")
def config4_weights(gpu_device):
  from lmoe import ops
  from lmoe.workloads import random_mxfp4
  packed, scale = random_mxfp4(1, 2048, 7168, gpu_device, seed=4)
  tpk, tsc = ops.mxfp4_tile_weights(packed, scale)
  pk, sc = to_np(packed), to_np(scale)
  wd = O.bf16_round(O.dequantize_mxfp4(pk[0], sc[0]))  # exact in bf16 for scales -8..2
  return packed, scale, tpk, tsc, pk, sc, wd


@pytest.mark.parametrize("m", CONFIG4_M)
def test_config4_mxfp4_matmul_full_size(gpu_device, config4_weights, m):
  """Every MXFP4 kernel at config 4: LDS dequant on checkpoint-layout and on
  tiled weights (split-K where the default picks it, M <= 1024, and
  unsplit), the skinny kernel (M <= 128), and the native scaled MFMA (MXFP8
  activations) against its own exact oracle."""
  from lmoe import ops
  packed, scale, tpk, tsc, pk, sc, wd = config4_weights
  rng = np.random.default_rng(40 + m)
  a = O.bf16_round(rng.standard_normal((m, 7168)))
  gs = np.array([m], np.int32)
  ref32 = np.matmul(a, wd.T, dtype=np.float32)
  ref = O.bf16_round(ref32)
  ad, gd = to_dev(a, "bf16"), to_dev(gs)
  errs = {}
  errs["checkpoint"] = max_rel(to_np(ops.ragged_dot_mxfp4(ad, packed, scale, gd)), ref)
  errs["tiled"] = max_rel(to_np(ops.ragged_dot_mxfp4(ad, tpk, tsc, gd, weight_layout="tiled")), ref)
  errs["tiled unsplit"] = max_rel(to_np(ops.ragged_dot_mxfp4(ad, tpk, tsc, gd, weight_layout="tiled", k_split=1)),
                                  ref)
  if m <= 128:
    errs["skinny"] = max_rel(to_np(ops.ragged_dot_mxfp4(ad, tpk, tsc, gd, weight_layout="tiled", mode="skinny",
                                                        max_group_rows=m)), ref)
  # scaled MFMA: activations quantised to MXFP8; f32 output against the exact
  # dot of the quantised operands, |d| <= 2^-14 sum|a w| elementwise
  codes, qs = O.quantize_mxfp8(a)
  q, qsd = ops.quantize_mxfp8(ad)
  out = to_np(ops.ragged_dot_mxfp8_mxfp4(q, qsd, tpk, tsc, gd, out_dtype=torch.float32))
  aq = O.dequantize_mxfp8(codes, qs).astype(np.float64)
  exact = aq @ wd.T.astype(np.float64)
  bound = 2.0 ** -14 * (np.abs(aq) @ np.abs(wd.T).astype(np.float64))
  viol = int((np.abs(out - exact) > bound).sum())
  dev_bf16 = max_rel(out, ref32)
  banner(f"config 4 M={m}: " + " ".join(f"{k} {v:.2e}" for k, v in errs.items())
         + f"; scaled-MFMA bound violations {viol}, deviation of MXFP8 activations from bf16 {dev_bf16:.2e}")
  for k, v in errs.items():
    assert v <= 2e-2, (k, v)
  assert viol == 0


def test_config5_layer_full_size(gpu_device):
  """The benchmarked configuration end to end at full size, every stage."""
  from lmoe.forward import LocalShardLatentMoE
  from lmoe.workloads import Config5, make_config5
  c = Config5()
  banner("config 5 full-size layer")
  hidden, w, experts = make_config5(gpu_device, c, "mxfp4")
  layer = LocalShardLatentMoE(c.config(), router_weight=w["router_weight"],
                              e_score_correction_bias=w["e_score_correction_bias"], down_proj=w["down_proj"],
                              up_proj=w["up_proj"], norm_scale=w["norm_scale"], local_expert_start=c.local_start,
                              local_num_experts=c.local_experts, expert_format="mxfp4", experts=experts,
                              capacity_factor=c.capacity_factor)
  out = layer.forward(hidden)
  out_st, st = layer.forward(hidden, return_stages=True)
  assert torch.equal(out, out_st)
  I = c.intermediate
  gu = O.dequantize_mxfp4(to_np(experts["gu_packed"]), to_np(experts["gu_scale"]))
  dn = O.dequantize_mxfp4(to_np(experts["down_packed"]), to_np(experts["down_scale"]))
  del experts
  gate, up, down = gu[:, :I, :].transpose(0, 2, 1), gu[:, I:, :].transpose(0, 2, 1), dn.transpose(0, 2, 1)
  wn = {k: to_np(v) for k, v in w.items()}
  check_single_shard("config 5 full size", to_np(hidden), wn, gate, up, down, c.config(), "bf16", c.local_start,
                     c.local_experts, c.capacity_factor, False, out, st)
