"""Seeded synthetic inputs for the BASELINE.json configurations, plus the OCP
MX (v1.0) MXFP4 weight quantiser used to produce MXFP4 expert weights.

Large tensors are generated with torch's Philox generator directly on the
target device (fast at 4096 x 7168); small ones may be generated on the CPU
and moved.  Every generator takes an explicit seed, so the same workload is
reproducible on any box.  These are benchmark inputs, not reference data.
"""

from __future__ import annotations

import dataclasses

import numpy as np
import torch

from .config import LatentMoEConfig

# ---------------------------------------------------------------------------
# MXFP4 quantisation (OCP Microscaling Formats v1.0, section 6.3)
# ---------------------------------------------------------------------------

_E2M1_MAG = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0)


def quantize_mxfp4(w: torch.Tensor, block: int = 32) -> tuple[torch.Tensor, torch.Tensor]:
  """w (..., N, K) float -> (packed (..., N, K/2) uint8, scale (..., N, K/block) uint8).

  Per block of ``block`` consecutive K elements: shared exponent
  X = floor(log2(amax)) - emax_elem (emax_elem = 2 for E2M1; an all-zero block
  uses amax = 1), clamped to [-127, 127] and stored as the E8M0 byte X + 127;
  elements are v / 2^X rounded to the nearest E2M1 value, ties to the even
  code, saturating at +-6.  Low nibble = element 2j, high nibble = 2j+1 (the
  checkpoint packing of mxfp4_dequant.py:14-17)."""
  *lead, n, k = w.shape
  if k % block or k % 2:
    raise ValueError(f"K={k} must be a multiple of {block}")
  x = w.float().reshape(*lead, n, k // block, block)
  amax = x.abs().amax(-1, keepdim=True)
  amax = torch.where(amax > 0, amax, torch.ones_like(amax))
  e = torch.floor(torch.log2(amax)) - 2.0
  e = e.clamp(-127.0, 127.0)
  q = x * torch.exp2(-e)
  a = q.abs()
  code = ((a > 0.25).to(torch.uint8) + (a >= 0.75).to(torch.uint8) + (a > 1.25).to(torch.uint8) +
          (a >= 1.75).to(torch.uint8) + (a > 2.5).to(torch.uint8) + (a >= 3.5).to(torch.uint8) +
          (a > 5.0).to(torch.uint8))
  code = code | (torch.signbit(q) & (code > 0)).to(torch.uint8) << 3
  code = code.reshape(*lead, n, k)
  packed = (code[..., 0::2] | (code[..., 1::2] << 4)).contiguous()
  scale = (e.squeeze(-1) + 127.0).to(torch.uint8).contiguous()
  return packed, scale


def random_mxfp4(g: int, n: int, k: int, device, seed: int, scale_lo: int = 119,
                 scale_hi: int = 129) -> tuple[torch.Tensor, torch.Tensor]:
  """BASELINE config 4 weights: codes uniform over the 16 E2M1 values (both
  nibbles of every byte uniform), scale exponents uniform in
  [scale_lo-127, scale_hi-127] (default -8..2)."""
  gen = torch.Generator(device=device).manual_seed(seed)
  packed = torch.randint(0, 256, (g, n, k // 2), generator=gen, device=device, dtype=torch.int32)
  scale = torch.randint(scale_lo, scale_hi + 1, (g, n, k // 32), generator=gen, device=device,
                        dtype=torch.int32)
  return packed.to(torch.uint8), scale.to(torch.uint8)


# ---------------------------------------------------------------------------
# Workloads
# ---------------------------------------------------------------------------


def zipf_group_sizes(m: int, g: int, seed: int, s: float = 1.1, n_zero: int = 3) -> np.ndarray:
  """BASELINE config 2 group sizes: multinomial(m, p) with p_g ~ (rank_g+1)^-s
  over a seeded permutation of ranks; n_zero seeded groups emptied into the
  largest remaining group (so sum == m)."""
  rng = np.random.default_rng(seed)
  rank = rng.permutation(g)
  p = (rank + 1.0) ** -s
  p /= p.sum()
  gs = rng.multinomial(m, p)
  zero = rng.choice(g, n_zero, replace=False)
  big = int(np.argmax(np.where(np.isin(np.arange(g), zero), -1, gs)))
  gs[big] += gs[zero].sum()
  gs[zero] = 0
  return gs.astype(np.int32)


# ---------------------------------------------------------------------------
# The reference's ragged_dot group-distribution matrix
# (05_ragged_dot_on_tpu/benchmark_harness.py:100-153): three shapes, five
# ways of splitting the M rows over the G groups.  The harness draws the sizes
# with tokamax.generate_ragged_dot_group_sizes (tokamax is not installed
# here); this restates its call contract -- an even split when p is None,
# otherwise M rows drawn over the groups with probabilities p -- as a seeded
# multinomial, so the probability vectors are the harness's own but the
# per-seed vectors are this generator's.
# ---------------------------------------------------------------------------

# name -> (M, K, N, G); the harness runs them in float32 (its ShapeCase
# default) and compares against a bf16 tolerance for bf16 inputs
HARNESS_SHAPES = {"small": (512, 256, 384, 4), "medium_a": (2048, 512, 512, 8), "medium_b": (4096, 1024, 1024, 16)}


def harness_distribution(name: str, g: int) -> list[float] | None:
  """The probability vector of one of the harness's distributions
  (benchmark_harness.py:116-150); None for "uniform" (an even split)."""
  if name == "uniform":
    return None
  if name == "mild_skew":  # group 0 gets about twice the average
    p = [1.0] * g
    p[0] = 2.0
  elif name == "heavy_skew":  # group 0 takes most of the rows
    p = [1.0] * g
    p[0] = float(g)
  elif name == "empty_groups":  # the second half of the groups gets nothing
    half = max(g // 2, 1)
    p = [1.0] * half + [0.0] * (g - half)
  elif name == "single_dominant":  # every row in group 0
    p = [0.0] * g
    p[0] = 1.0
  else:
    raise ValueError(f"distribution {name!r}")
  s = sum(p)
  return [x / s for x in p]


HARNESS_DISTRIBUTIONS = ("uniform", "mild_skew", "heavy_skew", "empty_groups", "single_dominant")


def harness_group_sizes(m: int, g: int, dist: str, seed: int = 0) -> np.ndarray:
  """int32 group sizes summing to m: an even split (the first m % g groups one
  row larger) for "uniform", a seeded multinomial over the distribution's
  probabilities otherwise."""
  p = harness_distribution(dist, g)
  if p is None:
    gs = np.full(g, m // g, np.int64)
    gs[: m % g] += 1
  else:
    gs = np.random.default_rng(seed).multinomial(m, p)
  return gs.astype(np.int32)


def _normal(shape, std, gen, device, dtype=torch.bfloat16):
  return (torch.randn(shape, generator=gen, device=device, dtype=torch.float32) * std).to(dtype)


@dataclasses.dataclass
class Config5:
  """full local-shard LatentMoE forward."""
  tokens: int = 4096
  hidden: int = 7168
  latent: int = 1024
  intermediate: int = 2048
  experts: int = 896
  top_k: int = 16
  local_start: int = 0
  local_experts: int = 112
  capacity_factor: float = 2.0
  zipf_skew: float = 1.2
  seed: int = 0

  def config(self) -> LatentMoEConfig:
    return LatentMoEConfig(hidden_size=self.hidden, latent_size=self.latent,
                           intermediate_size=self.intermediate, num_experts=self.experts,
                           top_k=self.top_k, num_shared_experts=0)


def make_config5(device, c: Config5 | None = None, expert_format: str = "mxfp4"):
  """Inputs and prepared weights of config 5.

  Router skew: the reference's only skew mechanism is e_score_correction_bias
  (selection-only, ref.py:350-352); BASELINE asks for "logits plus a Zipf(1.2)
  per-expert bias".  The bias is folded into the router *logits* by a seeded
  per-expert offset -1.2*ln(rank+1) added through an extra hidden feature:
  hidden[:, -1] = 1 and router_weight[-1, e] = offset_e, so the logits carry
  the skew and the combine weights see it (the "bias on logits" reading).
  Expert weights: N(0, 0.02^2) quantised to MXFP4 with the OCP rule.
  Returns (hidden, weights dict, experts dict) on ``device``."""
  c = c or Config5()
  gen = torch.Generator(device=device).manual_seed(c.seed)
  hidden = torch.randn((c.tokens, c.hidden), generator=gen, device=device).to(torch.bfloat16)
  router = _normal((c.hidden, c.experts), 0.02, gen, device)
  rng = np.random.default_rng(c.seed + 1)
  rank = rng.permutation(c.experts)
  offset = torch.from_numpy((-c.zipf_skew * np.log(rank + 1.0)).astype(np.float32)).to(device)
  hidden[:, -1] = 1.0
  router[-1, :] = offset.to(torch.bfloat16)
  w = {
      "router_weight": router,
      "e_score_correction_bias": torch.zeros(c.experts, device=device),
      "down_proj": _normal((c.hidden, c.latent), 0.02, gen, device),
      "up_proj": _normal((c.latent, c.hidden), 0.02, gen, device),
      "norm_scale": torch.ones(c.latent, device=device, dtype=torch.bfloat16),
  }
  L = c.local_experts
  experts = {}
  # gate/up as one [gate; up] (L+1, 2I, lat) matrix in checkpoint (out, in)
  # layout; the trailing expert is the zero padding bucket.
  gu = _normal((L + 1, 2 * c.intermediate, c.latent), 0.02, gen, device, torch.float32)
  gu[L] = 0
  dn = _normal((L + 1, c.latent, c.intermediate), 0.02, gen, device, torch.float32)
  dn[L] = 0
  if expert_format == "mxfp4":
    experts["gu_packed"], experts["gu_scale"] = _quantize_chunked(gu)
    experts["down_packed"], experts["down_scale"] = _quantize_chunked(dn)
  else:
    experts["gu_nk"] = gu.to(torch.bfloat16).contiguous()
    experts["down_nk"] = dn.to(torch.bfloat16).contiguous()
  del gu, dn
  return hidden, w, experts


def _quantize_chunked(w: torch.Tensor, chunk: int = 8):
  packs, scales = [], []
  for i in range(0, w.shape[0], chunk):
    p, s = quantize_mxfp4(w[i:i + chunk])
    packs.append(p)
    scales.append(s)
  return torch.cat(packs).contiguous(), torch.cat(scales).contiguous()


def routed_rows(topk_idx: torch.Tensor, start: int, L: int) -> int:
  """Number of (token, slot) assignments that land in [start, start+L)."""
  return int(((topk_idx >= start) & (topk_idx < start + L)).sum().item())


# ---------------------------------------------------------------------------
# BASELINE configs 1 and 3
# ---------------------------------------------------------------------------


def make_config1(seed: int = 0):
  """the reduced-scale fp32 layer the reference's naive CPU
  forward runs (ref.py:330-435): 128 tokens, d_model 256 -> latent 128, 8
  experts, top-2, expert FFN 128 -> 256 -> 128, one shared expert (the
  reference's small configs carry one, ref.py:174-188), activations N(0, 1),
  weights N(0, 0.02^2) from ``seed``, bias 0, norm scale 1.  Returns
  (config, hidden (128, 256) f32, weights dict of f32 numpy arrays in the
  reference (in, out) layout)."""
  cfg = LatentMoEConfig(hidden_size=256, latent_size=128, intermediate_size=256, num_experts=8, top_k=2,
                        num_shared_experts=1)
  rng = np.random.default_rng(seed)
  n = lambda *s: (rng.standard_normal(s) * 0.02).astype(np.float32)
  h, lat, inter, e = cfg.hidden_size, cfg.latent_size, cfg.intermediate_size, cfg.num_experts
  w = {
      "router_weight": n(h, e), "e_score_correction_bias": np.zeros(e, np.float32),
      "down_proj": n(h, lat), "up_proj": n(lat, h),
      "expert_gate": n(e, lat, inter), "expert_up": n(e, lat, inter), "expert_down": n(e, inter, lat),
      "norm_scale": np.ones(lat, np.float32),
      "shared_gate": n(h, inter), "shared_up": n(h, inter), "shared_down": n(inter, h),
  }
  hidden = rng.standard_normal((128, h)).astype(np.float32)
  return cfg, hidden, w


@dataclasses.dataclass
class Config3:
  """fused gate/up + SiTU-GLU + down on one GPU's shard."""
  tokens: int = 2048
  latent: int = 1024
  intermediate: int = 2048
  experts: int = 896
  top_k: int = 16
  local_start: int = 0
  local_experts: int = 112
  capacity_factor: float = 2.0
  seed: int = 0

  def config(self) -> LatentMoEConfig:
    return LatentMoEConfig(hidden_size=self.latent, latent_size=self.latent,
                           intermediate_size=self.intermediate, num_experts=self.experts,
                           top_k=self.top_k, num_shared_experts=0)


def make_config3(device, c: Config3 | None = None):
  """Inputs of config 3: router logits N(0, 1) f32 (T, E) *given* (seeded
  numpy), x N(0, 1) bf16 (T, lat), and the shard's expert weights in the
  reference (G, K, N) layout, N(0, 0.02^2) bf16, L + 1 groups (the trailing
  padding bucket is zero).  Returns (logits, x, gate, up, down)."""
  c = c or Config3()
  rng = np.random.default_rng(c.seed)
  logits = torch.from_numpy(rng.standard_normal((c.tokens, c.experts)).astype(np.float32)).to(device)
  gen = torch.Generator(device=device).manual_seed(c.seed + 1)
  x = torch.randn((c.tokens, c.latent), generator=gen, device=device).to(torch.bfloat16)
  L = c.local_experts

  def stack(k, n):
    w = _normal((L + 1, k, n), 0.02, gen, device)
    w[L] = 0
    return w

  gate = stack(c.latent, c.intermediate)
  up = stack(c.latent, c.intermediate)
  down = stack(c.intermediate, c.latent)
  return logits, x, gate, up, down


# ---------------------------------------------------------------------------
# a20: generate_local_shard_workload (ref.py:474-598)
# ---------------------------------------------------------------------------


def _draw_global_picks(rng: np.random.Generator, num_tokens: int, global_num_experts: int,
                       top_k: int) -> np.ndarray:
  """(num_tokens, top_k) expert ids, each row top_k distinct ids drawn
  uniformly without replacement (the first top_k positions of a uniformly
  random permutation, from the ranks of i.i.d. uniforms)."""
  keys = rng.random((num_tokens, global_num_experts))
  return np.argsort(keys, axis=1, kind="stable")[:, :top_k].astype(np.int32)


def generate_local_shard_workload(num_tokens: int, global_num_experts: int, top_k: int,
                                  local_num_experts: int, latent_size: int,
                                  dtype: torch.dtype = torch.bfloat16, capacity_factor: float = 2.0,
                                  tile_size: int = 128, *, seed: int = 0, device="cuda"):
  """``generate_local_shard_workload`` (ref.py:474-598): a synthetic expert
  shard input under a uniform, untrained top-k-of-E router.

  Each token draws ``top_k`` distinct experts uniformly from
  ``global_num_experts``; only picks below ``local_num_experts`` are kept (by
  symmetry, any block of ``local_num_experts`` ids would do).  Kept picks are
  stable-sorted by expert id.  ``m_padded`` = round_up(ceil(T*k*L/E * cf),
  tile), the ceil taken on the f32 value as ``jnp.ceil`` does (ref.py:568);
  picks past ``m_padded`` (aggregate overflow) are dropped from the tail of
  the sorted order with a warning printed, as in the reference.  The real
  per-expert counts are left as drawn; one trailing padding bucket brings
  the total to ``m_padded``.

  Returns (sorted_tokens (m_padded, latent) ``dtype`` with N(0, 1) rows for
  kept picks and zero padding rows, group_sizes (L+1,) int32, valid_mask
  (m_padded,) bool, per_expert_counts (L,) int32), all on ``device``.  The
  draw is seeded (numpy PCG64 for the routing, torch's generator on
  ``device`` for the token rows), so it is reproducible but not the JAX
  PRNG stream of the reference."""
  rng = np.random.default_rng(seed)
  picks = _draw_global_picks(rng, num_tokens, global_num_experts, top_k).reshape(-1)
  local_ids = np.sort(picks[picks < local_num_experts], kind="stable")
  num_raw = local_ids.shape[0]
  expected_total = num_tokens * top_k * local_num_experts / global_num_experts
  m_padded = -(-int(np.ceil(np.float32(expected_total * capacity_factor))) // tile_size) * tile_size
  if num_raw > m_padded:
    print(f"[shard-workload] WARNING: m_padded={m_padded} overflowed by the total draw -- dropping "
          f"{num_raw - m_padded} of {num_raw} raw assignments from the tail of the expert-sorted order "
          "(raise capacity_factor if this matters for the benchmark)")
    local_ids = local_ids[:m_padded]
  keep = local_ids.shape[0]
  counts = np.bincount(local_ids, minlength=local_num_experts).astype(np.int32)
  group_sizes = np.concatenate([counts, np.array([m_padded - keep], np.int32)])
  gen = torch.Generator(device=device).manual_seed(seed + 1)
  sorted_tokens = torch.zeros((m_padded, latent_size), dtype=dtype, device=device)
  if keep:
    sorted_tokens[:keep] = torch.randn((keep, latent_size), generator=gen, device=device).to(dtype)
  valid = torch.zeros(m_padded, dtype=torch.bool, device=device)
  valid[:keep] = True
  return (sorted_tokens, torch.from_numpy(group_sizes).to(device), valid,
          torch.from_numpy(counts).to(device))
