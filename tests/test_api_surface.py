"""Reference names a caller of the hot path may import, beyond the kernels'
own entry points: ``init_weights`` (ref.py:255-283), the naive shard FFN's
name ``_local_shard_expert_ffn`` (ref.py:1486-1528), and the tile helpers
``_round_up_to_tile`` / ``_MOSAIC_TILE_SIZE`` (ref.py:149-153).  CPU checks:
shapes, dtypes and the weight law; seeding; the FFN name issuing the same
library calls as its ragged_dot form (recording stand-in library)."""
import numpy as np
import pytest
import torch

import _stand_in
from lmoe import config as C
from lmoe import forward, ops


@pytest.mark.parametrize("cfg", [C.toy_config(), C.mosaic_correctness_config()])
def test_init_weights_shapes_dtypes_and_law(cfg):
  w = C.init_weights(cfg, 3, torch.bfloat16, device="cpu")
  h, lat, inter, e, ns = (cfg.hidden_size, cfg.latent_size, cfg.intermediate_size, cfg.num_experts,
                          cfg.num_shared_experts)
  want = {"router_weight": (h, e), "e_score_correction_bias": (e,), "down_proj": (h, lat), "up_proj": (lat, h),
          "expert_gate": (e, lat, inter), "expert_up": (e, lat, inter), "expert_down": (e, inter, lat),
          "norm_scale": (lat,), "shared_gate": (h, inter * ns), "shared_up": (h, inter * ns),
          "shared_down": (inter * ns, h)}
  for name, shape in want.items():
    t = getattr(w, name)
    assert tuple(t.shape) == shape and t.dtype == torch.bfloat16, name
  assert not w.e_score_correction_bias.any() and bool((w.norm_scale == 1).all())
  # every matrix N(0, 0.02^2): the pooled sample's mean and spread
  pooled = torch.cat([getattr(w, n).float().reshape(-1) for n in want if n not in ("e_score_correction_bias",
                                                                                     "norm_scale")])
  n = pooled.numel()
  assert abs(float(pooled.mean())) < 5 * 0.02 / np.sqrt(n)
  assert abs(float(pooled.std()) / 0.02 - 1) < 0.02


def test_init_weights_seeding():
  cfg = C.toy_config()
  a, b = C.init_weights(cfg, 7, device="cpu"), C.init_weights(cfg, 7, device="cpu")
  c = C.init_weights(cfg, 8, device="cpu")
  assert torch.equal(a.expert_up, b.expert_up) and not torch.equal(a.expert_up, c.expert_up)
  assert a.router_weight.dtype == torch.float32
  g = torch.Generator().manual_seed(7)
  assert torch.equal(C.init_weights(cfg, g, device="cpu").router_weight, a.router_weight)


def test_tile_helpers_under_the_reference_names():
  assert ops._MOSAIC_TILE_SIZE == 128
  assert [ops._round_up_to_tile(v) for v in (0, 1, 128, 129)] == [0, 128, 128, 256]
  assert ops._round_up_to_tile(5, 4) == 8


def test_naive_ffn_name_runs_the_grouped_gemms(monkeypatch):
  rec = _stand_in.install(monkeypatch)
  cfg = C.mosaic_correctness_config()
  w = C.init_weights(cfg, 1, torch.bfloat16, device="cpu")
  gs = torch.tensor([40, 0, 30, 58], dtype=torch.int32)
  x = torch.randn(128, cfg.latent_size).to(torch.bfloat16)
  args = (x, w.expert_gate[:4].contiguous(), w.expert_up[:4].contiguous(), w.expert_down[:4].contiguous(), gs, cfg)
  ops._local_shard_expert_ffn(*args)
  naive = rec.names()
  rec.calls.clear()
  ops._local_shard_expert_ffn_ragged_dot(*args)
  assert naive == rec.names() == ["lmoe_ragged_dot", "lmoe_ragged_dot", "lmoe_situ_and_mul", "lmoe_ragged_dot"]


def test_initialised_weights_drive_the_unsharded_forward(monkeypatch):
  """init_weights' output is what latent_moe_forward takes: the forward's
  host logic runs on it (CPU tensors, recording stand-in) up to its last
  library call."""
  rec = _stand_in.install(monkeypatch)
  cfg = C.mosaic_correctness_config()
  w = C.init_weights(cfg, 2, torch.bfloat16, device="cpu")
  hidden = torch.randn(16, cfg.hidden_size).to(torch.bfloat16)
  try:
    forward.latent_moe_forward(hidden, w, cfg)
  except IndexError:
    pass  # the stand-in writes no top-k ids; the host-side gather past them reads garbage
  assert "lmoe_router_topk_ld" in rec.names()
