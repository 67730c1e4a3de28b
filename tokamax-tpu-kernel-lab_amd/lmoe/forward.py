"""LatentMoE forwards on the HIP kernels, keeping the reference's entry points.

* ``latent_moe_forward`` / ``latent_moe_forward_ragged_dot`` -- the unsharded
  8-step forward (ref.py:330-435, rd.py:317-391): dispatch over all E experts,
  f32 weighted combine.
* ``latent_moe_forward_ragged_dot_single_shard_jittable`` -- one local shard
  as the whole routed population (rd.py:1035-1137), the production path.
* ``LocalShardLatentMoE`` -- the same single-shard forward on weights prepared
  once (k-contiguous bf16 or MXFP4 checkpoint layout), used by the benchmark.

ref.py = 05_ragged_dot_on_tpu/kimi_k3_latent_moe_reference.py,
rd.py = 05_ragged_dot_on_tpu/kimi_k3_latent_moe_ragged_dot.py.
"""

from __future__ import annotations

import torch

from . import ops
from .config import LatentMoEConfig, LatentMoEWeights


def _stage_order_from_slot_pos(slot_pos: torch.Tensor, m: int) -> torch.Tensor:
  """Dispatch permutation (row -> flat slot) from its inverse, for reporting."""
  order = torch.full((m,), -1, dtype=torch.int64, device=slot_pos.device)
  s = torch.arange(slot_pos.numel(), device=slot_pos.device)
  keep = slot_pos >= 0
  order[slot_pos[keep].long()] = s[keep]
  return order


def latent_moe_forward(hidden_states: torch.Tensor, weights: LatentMoEWeights, config: LatentMoEConfig,
                       act: str = "sigmoid", return_intermediates: bool = False,
                       implementation: str | None = None):
  """Unsharded forward, ref.py:330-435.  Gate math in f32, combine weight kept
  f32 through the weighted sum (ref.py:357-361, 413-416)."""
  if implementation not in (None, "hip"):
    raise NotImplementedError(f"implementation={implementation!r}")
  W = weights
  t = hidden_states.shape[0]
  k, e = config.top_k, config.num_experts
  b, bl = config.activation_situ_beta, config.activation_situ_linear_beta
  logits = ops.router_logits(hidden_states, W.router_weight)
  idx, w, scores = ops.router_topk_from_logits(logits, W.e_score_correction_bias, k, config.moe_renormalize,
                                               config.routed_scaling_factor, act, torch.float32,
                                               return_scores=True)
  x = ops.dense(hidden_states, W.down_proj)
  d = ops.dispatch_local(idx, w, x, 0, e, t * k)  # every slot kept: no truncation, empty pad group
  gs = d.group_sizes[:e]
  gate = ops.ragged_dot(d.sorted_tokens, W.expert_gate, gs)
  up = ops.ragged_dot(d.sorted_tokens, W.expert_up, gs)
  situ = ops._situ_and_mul(gate, up, b, bl)
  down = ops.ragged_dot(situ, W.expert_down, gs)
  routed = ops.combine_slots(down, d.slot_pos, w, t, k, mode="slot_sum", out_dtype=hidden_states.dtype)
  normed = ops._rms_norm(routed, W.norm_scale, config.rms_norm_eps)
  up_out = ops.dense(normed, W.up_proj)
  shared = ops._situ_glu_mlp(hidden_states, W.shared_gate, W.shared_up, W.shared_down, b, bl)
  final = ops.add(up_out, shared)
  if not return_intermediates:
    return final
  bias = W.e_score_correction_bias
  inter = {
      "router_logits": logits,
      "router_scores_before_bias": scores,
      "router_scores_for_choice": scores + (bias.float() if bias is not None else 0.0),
      "topk_indices": idx,
      "topk_weights": w,
      "latent_projection": x,
      "sorted_token_indices": _stage_order_from_slot_pos(d.slot_pos, t * k),
      "group_sizes": gs,
      "expert_gate_output": gate,
      "expert_up_output": up,
      "situ_output": situ,
      "expert_down_output": down,
      "routed_output_before_combine": down[d.slot_pos.long()],
      "routed_output_after_combine": routed,
      "normalized_output": normed,
      "up_projection_output": up_out,
      "shared_expert_output": shared,
      "final_output": final,
  }
  return final, inter


def latent_moe_forward_ragged_dot(hidden_states, weights, config, implementation=None, **kw):
  """rd.py:317-391 -- the same forward with the expert FFN as three ragged_dots."""
  return latent_moe_forward(hidden_states, weights, config, implementation=implementation, **kw)


def latent_moe_forward_ragged_dot_single_shard_jittable(
    hidden_states, router_weight, e_score_correction_bias, down_proj, shard_expert_gate,
    shard_expert_up, shard_expert_down, norm_scale, up_proj, shared_gate, shared_up, shared_down,
    config: LatentMoEConfig, local_expert_start: int, local_num_experts: int,
    capacity_factor: float = 2.0, implementation: str | None = None, act: str = "sigmoid",
    return_stages: bool = False, fused_gateup: bool = False):
  """rd.py:1035-1137.  shard_expert_* carry local_num_experts + 1 rows (the
  last is the padding bucket, computed as exact zeros without reading its
  weights).  shared_* may be None when the layer has no shared experts."""
  if implementation not in (None, "hip"):
    raise NotImplementedError(f"implementation={implementation!r}")
  t = hidden_states.shape[0]
  L = local_num_experts
  dt = hidden_states.dtype
  b, bl = config.activation_situ_beta, config.activation_situ_linear_beta
  x = ops.dense(hidden_states, down_proj)
  logits = ops.router_logits(hidden_states, router_weight)
  idx, w = ops.router_topk_from_logits(logits, e_score_correction_bias, config.top_k,
                                       config.moe_renormalize, config.routed_scaling_factor, act, dt)
  m_padded = ops.compute_m_padded(t, config.top_k, config.num_experts, L, capacity_factor)
  d = ops.dispatch_local(idx, w, x, local_expert_start, L, m_padded)
  if fused_gateup:
    shard_out = ops._local_shard_expert_ffn_ragged_dot_fused_gateup(
        d.sorted_tokens, shard_expert_gate, shard_expert_up, shard_expert_down, d.group_sizes, config,
        zero_group=L)
  else:
    shard_out = ops._local_shard_expert_ffn_ragged_dot(d.sorted_tokens, shard_expert_gate,
                                                       shard_expert_up, shard_expert_down,
                                                       d.group_sizes, config, zero_group=L)
  routed = ops.combine_slots(shard_out, d.slot_pos, d.padded_combine_weight, t, config.top_k,
                             mode="scatter_add", out_dtype=dt)
  normed = ops._rms_norm(routed, norm_scale, config.rms_norm_eps)
  up = ops.dense(normed, up_proj)
  if shared_gate is not None:
    shared = ops._situ_glu_mlp(hidden_states, shared_gate, shared_up, shared_down, b, bl)
    final = ops.add(up, shared)
  else:
    final = up
  if not return_stages:
    return final
  return final, {"x": x, "router_logits": logits, "topk_idx": idx, "topk_weight": w, "dispatch": d,
                 "shard_out": shard_out, "routed_out": routed, "normed": normed, "up": up}


class LocalShardLatentMoE:
  """Single-shard LatentMoE layer on weights prepared once.

  ``expert_format``: "bf16" (gate/up prefused to (L+1, 2I, K) and down to
  (L+1, lat, I), k-contiguous) or "mxfp4" (checkpoint layout: gate/up packed
  (L+1, 2I, lat/2) + scales (L+1, 2I, lat/32), down (L+1, lat, I/2) +
  (L+1, lat, I/32)).  Dense projections are stored (N, K).  Stages:
  router logits GEMM, down-projection GEMM, top-k, dispatch, fused gate/up +
  SiTU GEMM, down GEMM, combine, RMSNorm, up-projection GEMM (+ the shared
  expert MLP when given).

  ``shared``: the shared-expert MLP (ref.py:428-433) as {"gu_nk": (1, 2*SI,
  H) [gate | up] k-contiguous, "down_nk": (H, SI)}, i.e.
  ``ops.prefuse_gateup_weights_gnk(shared_gate[None], shared_up[None])`` and
  ``shared_down.t().contiguous()`` from the reference-layout weights.
  """

  def __init__(self, config: LatentMoEConfig, *, router_weight, e_score_correction_bias, down_proj,
               up_proj, norm_scale, local_expert_start: int, local_num_experts: int,
               expert_format: str, experts: dict, shared: dict | None = None,
               capacity_factor: float = 2.0, act: str = "sigmoid", mxfp4_mode: str = "lds_dequant",
               decode_tokens: int = 64):
    h, lat, e = config.hidden_size, config.latent_size, config.num_experts
    want = {"router_weight": (router_weight, (h, e)), "e_score_correction_bias": (e_score_correction_bias, (e,)),
            "down_proj": (down_proj, (h, lat)), "up_proj": (up_proj, (lat, h)), "norm_scale": (norm_scale, (lat,))}
    for name, (t, shape) in want.items():
      if tuple(t.shape) != shape:
        raise ValueError(f"{name} {tuple(t.shape)}: the config wants {shape}")
    if not (local_num_experts > 0 and 0 <= local_expert_start and local_expert_start + local_num_experts <= e):
      raise ValueError(f"local experts [{local_expert_start}, {local_expert_start + local_num_experts}) "
                       f"outside the {e} experts")
    if shared is not None:
      gu, dn = shared.get("gu_nk"), shared.get("down_nk")
      if (gu is None or dn is None or gu.dim() != 3 or gu.shape[0] != 1 or gu.shape[2] != h or gu.shape[1] % 2
          or tuple(dn.shape) != (h, gu.shape[1] // 2)):
        raise ValueError(f"shared: want gu_nk (1, 2*SI, {h}) and down_nk ({h}, SI), got "
                         f"{None if gu is None else tuple(gu.shape)} / {None if dn is None else tuple(dn.shape)}")
    if expert_format not in ("bf16", "mxfp4"):
      raise ValueError(f"expert_format={expert_format!r}: the layer takes 'bf16' or 'mxfp4' experts")
    if expert_format == "mxfp4" and mxfp4_mode not in ("lds_dequant", "scaled_mfma"):
      # the skinny decode kernel is chosen by size under "lds_dequant"; the
      # MXFP6 path has no fused SiTU epilogue for the gate/up GEMM
      raise NotImplementedError(f"mxfp4_mode={mxfp4_mode!r}: the layer runs 'lds_dequant' or 'scaled_mfma'")
    if expert_format == "mxfp4" and mxfp4_mode.startswith("scaled_mfma") and (
        lat % 128 or config.intermediate_size % 128):
      # the activations of both expert GEMMs are quantised in blocks of 128 along K
      raise NotImplementedError(f"mxfp4_mode={mxfp4_mode!r} needs latent and intermediate sizes that are "
                                f"multiples of 128 (got {lat}, {config.intermediate_size})")
    self.config = config
    self.L = local_num_experts
    self.start = local_expert_start
    self.cf = capacity_factor
    self.act = act
    self.expert_format = expert_format
    self.mxfp4_mode = mxfp4_mode
    # up to this many tokens the expert GEMMs run the skinny (decode) MXFP4
    # kernel: no local expert receives more than T rows (a token picks an
    # expert at most once), so a pass of up to T rows covers every group
    self.decode_tokens = decode_tokens
    self.router_nk = router_weight.t().contiguous()
    self.bias = e_score_correction_bias.float().contiguous()
    self.down_nk = down_proj.t().contiguous()
    # router logits and the down-projection read the same hidden states: one
    # GEMM over the concatenated (E + lat, H) weights (f32 out) replaces two,
    # reading the activations once; the latent columns are then rounded to
    # bf16, which is what the separate bf16 GEMM returns
    self.router_down_nk = None
    if self.router_nk.dtype == torch.bfloat16 and self.down_nk.dtype == torch.bfloat16:
      self.router_down_nk = torch.cat([self.router_nk, self.down_nk], 0).contiguous()
    self.up_nk = up_proj.t().contiguous()
    self.norm_scale = norm_scale.contiguous()
    self.experts = dict(experts)
    self.shared = shared
    # MXFP4 weights re-tiled once (k-step-major) so each k step's weight tile
    # streams into LDS as one contiguous read; the scaled-MFMA mode reads only
    # this layout
    self.weight_layout, self._sfx = "checkpoint", ""
    if expert_format == "mxfp4" and mxfp4_mode in ("lds_dequant", "scaled_mfma"):
      for w in ("gu", "down"):
        pk, sc = ops.mxfp4_tile_weights(experts[f"{w}_packed"], experts[f"{w}_scale"])
        self.experts[f"{w}_packed_tiled"], self.experts[f"{w}_scale_tiled"] = pk, sc
      self.weight_layout, self._sfx = "tiled", "_tiled"

  def _decode_path(self, t: int) -> bool:
    """Decode regime: few tokens, lds_dequant mode on tiled weights, shapes
    the skinny kernel takes (both expert GEMMs)."""
    if t > self.decode_tokens or self.mxfp4_mode != "lds_dequant" or self.weight_layout != "tiled":
      return False
    c = self.config
    return (ops.skinny_supported(c.latent_size, 2 * c.intermediate_size, self.L + 1, True)
            and ops.skinny_supported(c.intermediate_size, c.latent_size, self.L + 1, False))

  def _dense(self, x, w_nk, out_dtype=None):
    return ops.dense(x, w_nk, out_dtype=out_dtype, w_layout="nk")

  def forward(self, hidden: torch.Tensor, return_stages: bool = False, kernel_events: dict | None = None):
    """``kernel_events`` optionally maps a stage name ("gateup", "down") to a
    (start, end) pair of torch.cuda.Event recorded around that kernel on the
    current stream (used by the benchmark to time one kernel in place)."""
    c = self.config
    ev = kernel_events or {}
    t = hidden.shape[0]
    b, bl = c.activation_situ_beta, c.activation_situ_linear_beta
    m_padded = ops.compute_m_padded(t, c.top_k, c.num_experts, self.L, self.cf)
    decode = (self._decode_path(t) and hidden.dtype == torch.bfloat16
              and ops.small_dispatch_supported(t, c.top_k, c.latent_size, self.L, m_padded))
    x_src = None
    E = self.experts
    mx_mode, mx_kw = self.mxfp4_mode, {}
    if self.expert_format == "mxfp4" and self._decode_path(t):
      mx_mode, mx_kw = "skinny", {"max_group_rows": t}
    # Both paths below take the router top-k and the bf16 latent rows from one
    # launch over the fused router + down-projection output; it takes at most
    # 1024 latent columns (other sizes run the separate top-k and cast).
    proj_ok = (self.router_down_nk is not None
               and ops.router_topk_project_supported(self.router_nk.shape[0], c.latent_size))
    # Gathered rows (prefill, tiled MXFP4 experts, stages not returned): the
    # router launch also rounds the latent projection to bf16 (T rows), the
    # dispatch writes only its metadata, and the gate/up GEMM reads each
    # sorted row straight from its token's row -- no sorted_tokens copy.
    rows_path = (proj_ok and hidden.dtype == torch.bfloat16 and not return_stages
                 and self.expert_format == "mxfp4" and self.weight_layout == "tiled" and mx_mode == "lds_dequant")
    # Decode step (skinny expert GEMMs, stages not returned): the router launch
    # writes the bf16 token rows, and the one-launch dispatch runs inside the
    # skinny gate/up launch, which reads each sorted row's token row itself.
    fused_decode = (decode and mx_mode == "skinny" and not return_stages and proj_ok
                    and ops.dispatch_skinny_supported(t, c.top_k, c.latent_size, 2 * c.intermediate_size, self.L,
                                                      m_padded, True))
    act = None
    if fused_decode:
      e = self.router_nk.shape[0]
      rd = self._dense(hidden, self.router_down_nk, torch.float32)
      logits, x_src = rd[:, :e], rd[:, e:]
      idx, w, x = ops.router_topk_project(logits, x_src, self.bias, c.top_k, c.moe_renormalize,
                                          c.routed_scaling_factor, self.act, hidden.dtype)
      if "gateup" in ev:
        ev["gateup"][0].record()
      d, act = ops.dispatch_ragged_dot_mxfp4_skinny(idx, w, x, self.start, self.L, m_padded,
                                                    E["gu_packed" + self._sfx], E["gu_scale" + self._sfx],
                                                    fuse_gateup_activation=f"situ:{b}:{bl}",
                                                    skip_zero_group_rows=True)
    elif rows_path:
      e = self.router_nk.shape[0]
      rd = self._dense(hidden, self.router_down_nk, torch.float32)
      logits, x_src = rd[:, :e], rd[:, e:]
      idx, w, x = ops.router_topk_project(logits, x_src, self.bias, c.top_k, c.moe_renormalize,
                                          c.routed_scaling_factor, self.act, hidden.dtype)
      d = ops.dispatch_local(idx, w, None, self.start, self.L, m_padded, gather_rows=False, lat=c.latent_size)
      if "gateup" in ev:
        ev["gateup"][0].record()
      try:
        act = ops.ragged_dot_mxfp4(x, E["gu_packed" + self._sfx], E["gu_scale" + self._sfx], d.group_sizes,
                                   fuse_gateup_activation=f"situ:{b}:{bl}", mode=mx_mode, zero_group=self.L,
                                   weight_layout=self.weight_layout, skip_zero_group_rows=True,
                                   lhs_row_index=d.padded_token_idx)
      except NotImplementedError:
        # the streamed kernel does not take this size: gather the rows
        d = ops.dispatch_local(idx, w, x, self.start, self.L, m_padded, path="sort", skip_padding_rows=True)
    else:
      if self.router_down_nk is not None and hidden.dtype == torch.bfloat16:
        e = self.router_nk.shape[0]
        rd = self._dense(hidden, self.router_down_nk, torch.float32)
        logits = rd[:, :e]
        # the dispatch rounds the f32 latent rows to bf16 as it gathers them:
        # no separate cast (x itself is materialised only for the stages)
        x_src = rd[:, e:]
        x = ops.cast_rows(x_src, hidden.dtype) if return_stages else None
      else:
        logits = self._dense(hidden, self.router_nk, torch.float32)
        x = self._dense(hidden, self.down_nk)
      idx, w = ops.router_topk_from_logits(logits, self.bias, c.top_k, c.moe_renormalize,
                                           c.routed_scaling_factor, self.act, hidden.dtype)
      # padding rows of the sorted tokens are read by no later stage (the MXFP4
      # expert GEMMs skip the padding bucket) unless the stages are returned
      skip = self.expert_format == "mxfp4" and not return_stages
      d = ops.dispatch_local(idx, w, x_src if x_src is not None else x, self.start, self.L, m_padded,
                             path="small" if decode else "sort", skip_padding_rows=skip)
      if "gateup" in ev:
        ev["gateup"][0].record()
    if act is None and self.expert_format == "mxfp4":
      # padding-bucket rows (zero_group L) are never read downstream: left
      # unwritten unless the stages are returned
      act = ops.ragged_dot_mxfp4(d.sorted_tokens, E["gu_packed" + self._sfx], E["gu_scale" + self._sfx],
                                 d.group_sizes,
                                 fuse_gateup_activation=f"situ:{b}:{bl}", mode=mx_mode,
                                 zero_group=self.L, weight_layout=self.weight_layout,
                                 skip_zero_group_rows=not return_stages, **mx_kw)
    elif act is None:
      act = ops.ragged_dot_gateup_situ(d.sorted_tokens, E["gu_nk"], d.group_sizes, b, bl,
                                       rhs_layout="gnk", zero_group=self.L)
    if "gateup" in ev:
      ev["gateup"][1].record()
    if "down" in ev:
      ev["down"][0].record()
    if self.expert_format == "mxfp4":
      shard_out = ops.ragged_dot_mxfp4(act, E["down_packed" + self._sfx], E["down_scale" + self._sfx],
                                       d.group_sizes,
                                       mode=mx_mode, zero_group=self.L,
                                       weight_layout=self.weight_layout,
                                       skip_zero_group_rows=not return_stages, **mx_kw)
    else:
      shard_out = ops.ragged_dot(act, E["down_nk"], d.group_sizes, rhs_layout="gnk", zero_group=self.L)
    if "down" in ev:
      ev["down"][1].record()
    if ops.combine_rms_norm_supported(shard_out.shape[-1]):
      # combine and RMSNorm in one pass; the routed rows are materialised only
      # when the stages are returned
      res = ops.combine_slots_rms_norm(shard_out, d.slot_pos, d.padded_combine_weight, t, c.top_k,
                                       self.norm_scale, c.rms_norm_eps, mode="scatter_add", out_dtype=hidden.dtype,
                                       return_routed=return_stages)
      normed, routed = res if return_stages else (res, None)
    else:
      routed = ops.combine_slots(shard_out, d.slot_pos, d.padded_combine_weight, t, c.top_k,
                                 mode="scatter_add", out_dtype=hidden.dtype)
      normed = ops._rms_norm(routed, self.norm_scale, c.rms_norm_eps)
    out = self._dense(normed, self.up_nk)
    if self.shared is not None:
      S = self.shared
      sact = ops.ragged_dot_gateup_situ(hidden, S["gu_nk"], ops._ones_group(t, hidden.device), b, bl,
                                        rhs_layout="gnk")
      out = ops.add(out, self._dense(sact, S["down_nk"]))
    if not return_stages:
      return out
    return out, {"router_logits": logits, "x": x, "topk_idx": idx, "topk_weight": w, "dispatch": d,
                 "act": act, "shard_out": shard_out, "routed_out": routed, "normed": normed}
