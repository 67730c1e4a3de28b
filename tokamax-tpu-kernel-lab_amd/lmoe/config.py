"""Configuration and weight containers mirroring the reference's L2 types.

``LatentMoEConfig`` mirrors ``LatentMoEConfig`` (reference
05_ragged_dot_on_tpu/kimi_k3_latent_moe_reference.py:156-171) field for field,
with the same presets (``toy_config`` 174-188, ``kimi_k3_config`` 191-208,
``mosaic_correctness_config`` kimi_k3_latent_moe_ragged_dot.py:462-482,
``single_chip_kimi_k3_config`` kimi_k3_latent_moe_ragged_dot.py:500-533).

``LatentMoEWeights`` mirrors ``LatentMoEWeights`` (ref.py:217-252): the same
eleven fields in the same (in, out) layout (``x @ W``), held as torch tensors
on the device.  The expert stacks may be sliced to one shard of
``local_num_experts + 1`` rows (the trailing row is the padding bucket), as
the reference's single-shard forward expects (rd.py:1035-1137).
"""

from __future__ import annotations

import dataclasses
from typing import Any


@dataclasses.dataclass(frozen=True)
class LatentMoEConfig:
  hidden_size: int
  latent_size: int
  intermediate_size: int
  num_experts: int
  top_k: int
  num_shared_experts: int
  moe_renormalize: bool = True
  routed_scaling_factor: float = 1.0
  rms_norm_eps: float = 1e-5
  activation_situ_beta: float = 4.0
  activation_situ_linear_beta: float = 25.0


def toy_config() -> LatentMoEConfig:
  """ref.py:174-188 (dimension-matched to the small golden bundles)."""
  return LatentMoEConfig(hidden_size=64, latent_size=32, intermediate_size=48, num_experts=8,
                         top_k=2, num_shared_experts=1)


def kimi_k3_config() -> LatentMoEConfig:
  """ref.py:191-208."""
  return LatentMoEConfig(hidden_size=7168, latent_size=3584, intermediate_size=3072,
                         num_experts=896, top_k=16, num_shared_experts=2)


def mosaic_correctness_config() -> LatentMoEConfig:
  """rd.py:462-482 (dimension-matched to the mosaic golden bundles)."""
  return LatentMoEConfig(hidden_size=256, latent_size=128, intermediate_size=128, num_experts=8,
                         top_k=2, num_shared_experts=1)


def single_chip_kimi_k3_config(num_experts: int = 64) -> LatentMoEConfig:
  """rd.py:500-533."""
  return dataclasses.replace(kimi_k3_config(), num_experts=num_experts)


def config_from_official(official: dict) -> LatentMoEConfig:
  """Official config.json field names -> LatentMoEConfig (the field map of the
  reference's test_jax_reference_against_pytorch_golden.py:116-137)."""
  return LatentMoEConfig(
      hidden_size=official["hidden_size"],
      latent_size=official["routed_expert_hidden_size"],
      intermediate_size=official["moe_intermediate_size"],
      num_experts=official["num_experts"],
      top_k=official["num_experts_per_token"],
      num_shared_experts=official["num_shared_experts"],
      moe_renormalize=official["moe_renormalize"],
      routed_scaling_factor=official["routed_scaling_factor"],
      rms_norm_eps=official["rms_norm_eps"],
      activation_situ_beta=official["activation_situ_beta"],
      activation_situ_linear_beta=official["activation_situ_linear_beta"],
  )


WEIGHT_FIELDS = (
    "router_weight",  # (hidden, E)
    "e_score_correction_bias",  # (E,)
    "down_proj",  # (hidden, latent)
    "up_proj",  # (latent, hidden)
    "expert_gate",  # (E or L+1, latent, inter)
    "expert_up",  # (E or L+1, latent, inter)
    "expert_down",  # (E or L+1, inter, latent)
    "norm_scale",  # (latent,)
    "shared_gate",  # (hidden, inter*ns)
    "shared_up",  # (hidden, inter*ns)
    "shared_down",  # (inter*ns, hidden)
)


@dataclasses.dataclass(frozen=True)
class LatentMoEWeights:
  router_weight: Any
  e_score_correction_bias: Any
  down_proj: Any
  up_proj: Any
  expert_gate: Any
  expert_up: Any
  expert_down: Any
  norm_scale: Any
  shared_gate: Any
  shared_up: Any
  shared_down: Any

  def as_dict(self) -> dict:
    return {f: getattr(self, f) for f in WEIGHT_FIELDS}


def init_weights(config: LatentMoEConfig, key=0, dtype=None, device="cuda") -> LatentMoEWeights:
  """``init_weights`` (ref.py:255-283): every field in the (in, out) layout
  with the reference's shapes and law -- each matrix N(0, 0.02^2), the
  correction bias zero, the norm scale one, the shared-expert matrices
  (hidden, intermediate * num_shared_experts) / transposed -- as torch
  tensors of ``dtype`` (default float32) on ``device``.  ``key`` is an int
  seed or a torch.Generator; the reference's JAX PRNG stream is not
  reproduced (no expected output depends on the particular draws)."""
  import torch
  dtype = dtype or torch.float32
  gen = key if isinstance(key, torch.Generator) else torch.Generator(device=device).manual_seed(int(key))
  h, lat, inter, e = config.hidden_size, config.latent_size, config.intermediate_size, config.num_experts
  shared = inter * config.num_shared_experts

  def normal(*shape):
    return (torch.randn(shape, generator=gen, device=gen.device) * 0.02).to(device=device, dtype=dtype)

  return LatentMoEWeights(
      router_weight=normal(h, e), e_score_correction_bias=torch.zeros(e, dtype=dtype, device=device),
      down_proj=normal(h, lat), up_proj=normal(lat, h), expert_gate=normal(e, lat, inter),
      expert_up=normal(e, lat, inter), expert_down=normal(e, inter, lat),
      norm_scale=torch.ones(lat, dtype=dtype, device=device), shared_gate=normal(h, shared),
      shared_up=normal(h, shared), shared_down=normal(shared, h))


def weights_from_official_state_dict(sd: dict, config: LatentMoEConfig) -> dict:
  """Official (out, in) nn.Linear layout -> reference (in, out) layout, with the
  per-expert stacking of test_jax_reference_against_pytorch_golden.py:139-170
  (w1 = gate, w3 = up, w2 = down).  Works on numpy arrays; returns a dict keyed
  like ``LatentMoEWeights``."""
  import numpy as np
  e = config.num_experts
  return {
      "router_weight": np.ascontiguousarray(sd["gate.weight"].T),
      "e_score_correction_bias": np.asarray(sd["gate.e_score_correction_bias"]),
      "down_proj": np.ascontiguousarray(sd["routed_expert_down_proj.weight"].T),
      "up_proj": np.ascontiguousarray(sd["routed_expert_up_proj.weight"].T),
      "expert_gate": np.stack([sd[f"experts.{i}.w1.weight"].T for i in range(e)]),
      "expert_up": np.stack([sd[f"experts.{i}.w3.weight"].T for i in range(e)]),
      "expert_down": np.stack([sd[f"experts.{i}.w2.weight"].T for i in range(e)]),
      "norm_scale": np.asarray(sd["routed_expert_norm.weight"]),
      "shared_gate": np.ascontiguousarray(sd["shared_experts.gate_proj.weight"].T),
      "shared_up": np.ascontiguousarray(sd["shared_experts.up_proj.weight"].T),
      "shared_down": np.ascontiguousarray(sd["shared_experts.down_proj.weight"].T),
  }
