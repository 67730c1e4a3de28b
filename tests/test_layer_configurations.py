"""The local-shard layer across its configuration space, on the CPU: hidden,
latent and intermediate sizes, expert count, top-k, local expert range,
token count (none, decode and prefill), capacity factor (0 included),
expert format (MXFP4 or bf16), MXFP4 mode and stage return drawn by
hypothesis.  A configuration the
layer cannot run is refused when it is built (ValueError /
NotImplementedError); one it builds runs its forward against the recording
stand-in library without raising, every buffer it hands the library holds
what the call's sizes say, and (where no GPU is present) every call passes
the real library's host checks.  The forward chooses among several paths by
size (the one-launch decode dispatch, the gathered-rows gate/up, the fused
router projection, the stage-returning path); this checks that each
combination it can choose is one the library takes.  The reference-API
forwards (unsharded and functional single-shard) are swept the same way
over the configurations the reference allows."""

import pytest
import torch
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

import test_buffer_extents as X
from lmoe import _lib, forward, ops
from lmoe.workloads import Config5, make_config5

NO_GPU = torch.cuda.device_count() == 0


def _zero_config5(c, fmt):
  """``make_config5``'s shapes and dtypes, zero-filled: the recording stand-in
  computes nothing, so the values do not matter and drawing the random
  weights would take most of the sweep's time."""
  bf, u8, L, i2 = torch.bfloat16, torch.uint8, c.local_experts, 2 * c.intermediate
  z = torch.zeros
  w = {"router_weight": z(c.hidden, c.experts, dtype=bf), "e_score_correction_bias": z(c.experts),
       "down_proj": z(c.hidden, c.latent, dtype=bf), "up_proj": z(c.latent, c.hidden, dtype=bf),
       "norm_scale": torch.ones(c.latent, dtype=bf)}
  if fmt == "mxfp4":
    ex = {"gu_packed": z(L + 1, i2, c.latent // 2, dtype=u8), "gu_scale": z(L + 1, i2, c.latent // 32, dtype=u8),
          "down_packed": z(L + 1, c.latent, c.intermediate // 2, dtype=u8),
          "down_scale": z(L + 1, c.latent, c.intermediate // 32, dtype=u8)}
  else:
    ex = {"gu_nk": z(L + 1, i2, c.latent, dtype=bf), "down_nk": z(L + 1, c.latent, c.intermediate, dtype=bf)}
  return z(c.tokens, c.hidden, dtype=bf), w, ex


def _build(c, fmt, mode, zero_weights=False):
  hidden, w, ex = (_zero_config5 if zero_weights else lambda c, fmt: make_config5("cpu", c, fmt))(c, fmt)
  layer = forward.LocalShardLatentMoE(c.config(), router_weight=w["router_weight"],
                                      e_score_correction_bias=w["e_score_correction_bias"],
                                      down_proj=w["down_proj"], up_proj=w["up_proj"], norm_scale=w["norm_scale"],
                                      local_expert_start=c.local_start, local_num_experts=c.local_experts,
                                      expert_format=fmt, experts=ex, capacity_factor=c.capacity_factor,
                                      mxfp4_mode=mode)
  return layer, hidden


def _replay_refusals(calls):
  real = _lib.lib()
  out = []
  for name, args, _ in calls:
    rc = getattr(real, name)(*args)
    if rc not in (_lib.OK, _lib.ERR_HIP):
      out.append((name, rc, real.lmoe_last_error().decode()))
  return out


def test_configurations(monkeypatch):
  log = X.ExtentLog(monkeypatch)
  stats = {"ran": 0, "refused": 0}

  @settings(max_examples=120, deadline=None, derandomize=True, database=None,
            suppress_health_check=[HealthCheck.too_slow, HealthCheck.function_scoped_fixture])
  @given(st.data())
  def run(data):
    pick = lambda xs: data.draw(st.sampled_from(xs))
    e = pick([8, 16, 60, 128, 256])
    lat, inter = pick([64, 128, 192, 256, 1024, 1088, 2048]), pick([64, 128, 192, 256])
    L = pick([n for n in (1, 4, 15, 16, 60, 128) if n <= e])
    c = Config5(tokens=pick([0, 1, 2, 5, 16, 63, 64, 65, 200, 512]), hidden=pick([64, 128, 256]),
                latent=lat, intermediate=inter,
                experts=e, top_k=pick([k for k in (1, 2, 4, 8, 16) if k <= e]),
                local_start=pick(sorted({0, min(3, e - L), e - L})), local_experts=L,
                capacity_factor=pick([0.0, 1.0, 2.0, 4.0]))
    fmt = pick(["mxfp4", "mxfp4", "bf16"])
    mode = pick(["lds_dequant", "lds_dequant", "scaled_mfma"]) if fmt == "mxfp4" else "lds_dequant"
    stages = pick([False, False, True])
    try:
      layer, hidden = _build(c, fmt, mode, zero_weights=True)
    except (ValueError, NotImplementedError):
      stats["refused"] += 1
      return
    log.clear()
    layer.forward(hidden, return_stages=stages)  # a layer that builds runs
    X.check_extents(log.calls)
    if NO_GPU:
      assert not _replay_refusals(log.calls), (c, fmt, mode, stages)
    stats["ran"] += 1

  run()
  assert stats["ran"] >= 80, stats


def test_one_token_bf16_experts(monkeypatch):
  """One token through a layer with bf16 expert weights: the latent rows are
  a one-row slice of the fused router + down-projection output, rounded to
  bf16 by the dispatch as for any other batch (a single-row slice counts as
  contiguous to torch)."""
  log = X.ExtentLog(monkeypatch)
  c = Config5(tokens=1, hidden=128, latent=128, intermediate=64, experts=16, top_k=2, local_start=0,
              local_experts=16)
  layer, hidden = _build(c, "bf16", "lds_dequant")
  log.clear()
  layer.forward(hidden)
  assert "lmoe_ragged_dot_gateup_situ" in [n for n, _, _ in log.calls]


@pytest.mark.parametrize("t", [1, 2])
def test_dispatch_rounds_a_row_slice_to_bf16_at_every_batch_size(monkeypatch, t):
  X.ExtentLog(monkeypatch)
  wide = torch.zeros(t, 16 + 64)
  d = ops.dispatch_local(torch.zeros(t, 2, dtype=torch.int32), torch.zeros(t, 2), wide[:, 16:], 0, 4, 128,
                         path="sort")
  assert d.sorted_tokens.dtype == torch.bfloat16


def test_scaled_mode_refuses_sizes_it_cannot_quantise():
  c = Config5(tokens=4, hidden=128, latent=192, intermediate=128, experts=16, top_k=2, local_start=0,
              local_experts=16)
  with pytest.raises(NotImplementedError, match="multiples of 128"):
    _build(c, "mxfp4", "scaled_mfma")


@pytest.mark.parametrize("fmt,mode,error", [("mxfp4", "skinny", NotImplementedError),
                                            ("mxfp4", "scaled_mfma_fp6", NotImplementedError),
                                            ("mxfp4", "bogus", NotImplementedError), ("fp8", "lds_dequant", ValueError)])
def test_layer_refuses_modes_it_cannot_run(fmt, mode, error):
  """Expert formats and MXFP4 modes the layer has no forward for are refused
  when it is built (the skinny decode kernel is chosen by size, not by mode;
  the MXFP6 path has no fused SiTU epilogue for the gate/up GEMM)."""
  c = Config5(tokens=4, hidden=128, latent=128, intermediate=128, experts=16, top_k=2, local_start=0,
              local_experts=16)
  hidden, w, ex = make_config5("cpu", c, "mxfp4" if fmt == "mxfp4" else "bf16")
  with pytest.raises(error, match="mxfp4_mode" if fmt == "mxfp4" else "expert_format"):
    forward.LocalShardLatentMoE(c.config(), router_weight=w["router_weight"],
                                e_score_correction_bias=w["e_score_correction_bias"], down_proj=w["down_proj"],
                                up_proj=w["up_proj"], norm_scale=w["norm_scale"], local_expert_start=0,
                                local_num_experts=16, expert_format=fmt, experts=ex, mxfp4_mode=mode)


def test_reference_api_forwards(monkeypatch):
  """``latent_moe_forward`` (unsharded) and the functional single-shard
  forward across configurations the reference allows -- f32 or bf16
  weights, 1 to 128 experts, sizes off the 8-element grid (hidden 72,
  latent 24, intermediate 40), no / one / two shared experts, sigmoid or
  softmax gate, renormalised or not, fused gate/up or not: each runs without
  raising, with large-enough buffers and every call past the real library's
  host checks."""
  from lmoe.config import LatentMoEConfig, init_weights
  log = X.ExtentLog(monkeypatch)
  stats = {"ran": 0}

  @settings(max_examples=150, deadline=None, derandomize=True, database=None,
            suppress_health_check=[HealthCheck.too_slow, HealthCheck.function_scoped_fixture])
  @given(st.data())
  def run(data):
    pick = lambda xs: data.draw(st.sampled_from(xs))
    e = pick([1, 2, 8, 16, 60, 128])
    cfg = LatentMoEConfig(hidden_size=pick([8, 32, 48, 64, 72, 256]), latent_size=pick([8, 16, 24, 32, 48, 128]),
                          intermediate_size=pick([8, 16, 40, 48, 128]), num_experts=e,
                          top_k=pick([k for k in (1, 2, 4, 8, 16) if k <= e]), num_shared_experts=pick([0, 1, 2]),
                          moe_renormalize=pick([True, False]), routed_scaling_factor=pick([1.0, 2.5]))
    dt = pick([torch.float32, torch.bfloat16])
    W = init_weights(cfg, dtype=dt, device="cpu")
    h = torch.zeros(pick([0, 1, 2, 5, 20, 64, 300]), cfg.hidden_size, dtype=dt)
    act = pick(["sigmoid", "softmax"])
    log.clear()
    if pick(["unsharded", "shard"]) == "unsharded":
      forward.latent_moe_forward(h, W, cfg, act=act)
    else:
      L = pick([n for n in (1, 4, e) if n <= e])
      start = pick(sorted({0, e - L}))
      pad = lambda w: torch.cat([w[start:start + L], torch.zeros_like(w[:1])])
      forward.latent_moe_forward_ragged_dot_single_shard_jittable(
          h, W.router_weight, W.e_score_correction_bias, W.down_proj, pad(W.expert_gate), pad(W.expert_up),
          pad(W.expert_down), W.norm_scale, W.up_proj, W.shared_gate if cfg.num_shared_experts else None,
          W.shared_up, W.shared_down, cfg, start, L, capacity_factor=pick([0.0, 1.0, 2.0]), act=act,
          fused_gateup=pick([False, True]))
    X.check_extents(log.calls)
    if NO_GPU:
      assert not _replay_refusals(log.calls), (cfg, dt, h.shape)
    stats["ran"] += 1

  run()
  assert stats["ran"] == 150
